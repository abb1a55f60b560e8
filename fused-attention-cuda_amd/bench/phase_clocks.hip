// phase_clocks -- the per-phase cycle budget of the stage-5 kernel (fa_s5_tuned), read from the
// kernel itself. This translation unit compiles the kernel header with FA_PHASE_CLOCKS defined, so
// every wave records s_memtime / s_memrealtime stamps of its phases (prologue, key walk, merge and
// epilogue) and the cycles it waits at the step barriers; the library (libfa_hip.so) is built
// without them. The tool times K back-to-back launches over 4 rotating input sets (the same
// kernels and tiles the library launches for the shapes below) and prints, from the last launch's
// stamps: the launch time, the workgroups' lifetime, dispatch spread and finish spread, the mean
// cycles of each phase, the cycles per key-tile step and the barrier wait per step, and the shader
// clock (s_memtime cycles over s_memrealtime's 100 MHz).
//
//   usage: phase_clocks [C64|C128|C128_causal|LONG|GPT_attn|all] [launches]
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#ifndef FA_PHASE_CLOCKS
#define FA_PHASE_CLOCKS 1
#endif
#include "attn_mfma16.h"

namespace {

#define CHECK(x)                                                                          \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      std::fprintf(stderr, "phase_clocks: %s at %s:%d\n", hipGetErrorString(e_), __FILE__, \
                   __LINE__);                                                             \
      std::exit(1);                                                                       \
    }                                                                                     \
  } while (0)

struct Shape {
  const char* name;
  int B, H, N, D, causal;
  bool bf16;
  fa::LaunchFn fn;  // the tile the library picks for this shape
  int br, bc, waves;
  float std;        // input scale (LONG: 0.5, as the benchmark)
};

const Shape kShapes[] = {
    {"C64", 2, 8, 2048, 64, 0, false, &fa::m16::launch<5, _Float16, 64, 4, 2, 64>, 128, 128, 8, 1.f},
    {"C128", 2, 8, 2048, 128, 0, false, &fa::m16::launch<5, _Float16, 128, 4, 2, 32>, 128, 64, 8, 1.f},
    // Causal C128: the library halves the height (BR 64 x BC 64, 512 workgroups issued tile-major).
    {"C128_causal", 2, 8, 2048, 128, 1, false, &fa::m16::launch<5, _Float16, 128, 2, 2, 32>, 64, 64, 4, 1.f},
    // LONG: BR 128 x BC 32, four waves, two workgroups per CU (the narrow D = 128 tile).
    {"LONG", 1, 16, 8192, 128, 1, true, &fa::m16::launch<5, __bf16, 128, 4, 1, 32>, 128, 32, 4, 0.5f},
    // GPT-2 attention shape: BR 64 x BC 64, four waves (the short-walk D = 64 tile).
    {"GPT_attn", 8, 12, 1024, 64, 1, false, &fa::m16::launch<5, _Float16, 64, 2, 2, 32>, 64, 64, 4, 1.f},
};

template <typename T>
__global__ void fill(T* p, size_t n, uint32_t seed, float scale) {
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += gridDim.x * 256ull) {
    uint32_t h = static_cast<uint32_t>(i) * 0x9E3779B1u ^ seed;
    h ^= h >> 16;
    h *= 0x85EBCA6Bu;
    h ^= h >> 13;
    h *= 0xC2B2AE35u;
    h ^= h >> 16;
    // sum of two uniforms, centred: a bell-shaped value in (-1, 1)
    const float u = ((h & 0xFFFF) + (h >> 16)) * (1.0f / 65536.0f) - 1.0f;
    p[i] = static_cast<T>(1.7f * scale * u);
  }
}

void run(const Shape& s, int launches) {
  const size_t n = static_cast<size_t>(s.B) * s.H * s.N * s.D;
  // Rotating input sets: 4 (they stay in the 256 MB last-level cache), or PHASE_CLOCKS_SETS of
  // them, e.g. 32 at C64 (537 MB, twice that cache, as bench.py's cache-cold headline).
  const char* sets_env = std::getenv("PHASE_CLOCKS_SETS");
  const int kSets = sets_env != nullptr ? std::max(1, std::min(64, std::atoi(sets_env))) : 4;
  std::vector<void*> q(kSets), k(kSets), v(kSets), o(kSets);
  std::vector<float*> lse(kSets);
  for (int i = 0; i < kSets; ++i) {
    for (void** p : {&q[i], &k[i], &v[i], &o[i]}) CHECK(hipMalloc(p, n * 2));
    CHECK(hipMalloc(&lse[i], static_cast<size_t>(s.B) * s.H * s.N * 4));
    for (int t = 0; t < 3; ++t) {
      void* dst = t == 0 ? q[i] : t == 1 ? k[i] : v[i];
      if (s.bf16) {
        hipLaunchKernelGGL(fill<__bf16>, dim3(1024), dim3(256), 0, 0, static_cast<__bf16*>(dst), n,
                           3u * i + t + 1, s.std);
      } else {
        hipLaunchKernelGGL(fill<_Float16>, dim3(1024), dim3(256), 0, 0, static_cast<_Float16*>(dst),
                           n, 3u * i + t + 1, s.std);
      }
    }
  }
  auto args = [&](int i) {
    fa::KArgs a{};
    a.q = q[i];
    a.k = k[i];
    a.v = v[i];
    a.o = o[i];
    a.lse = lse[i];
    a.B = s.B;
    a.H = s.H;
    a.Hkv = s.H;
    a.N = s.N;
    a.scale = 1.0f / std::sqrt(static_cast<float>(s.D));
    a.c = a.scale * 1.44269504088896341f;
    a.causal = s.causal;
    a.qsb = a.ksb = a.vsb = a.osb = static_cast<long long>(s.H) * s.N * s.D;
    a.qsh = a.ksh = a.vsh = a.osh = static_cast<long long>(s.N) * s.D;
    a.qsn = a.ksn = a.vsn = a.osn = s.D;
    a.n_splits = 1;
    a.fd_h = fa::make_fastdiv(s.H);
    a.fd_group = fa::make_fastdiv(1);
    a.fd_splits = fa::make_fastdiv(1);
    return a;
  };
  hipStream_t st;
  CHECK(hipStreamCreate(&st));
  for (int i = 0; i < 20; ++i) CHECK(static_cast<hipError_t>(s.fn(args(i % kSets), st)));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0, st));
  for (int i = 0; i < launches; ++i) CHECK(static_cast<hipError_t>(s.fn(args(i % kSets), st)));
  CHECK(hipEventRecord(e1, st));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  const double us = 1000.0 * ms / launches;

  const int nwg = (s.N / s.br) * s.B * s.H;
  std::vector<unsigned long long> h(static_cast<size_t>(nwg) * 16 * 8);
  CHECK(hipMemcpyFromSymbol(h.data(), HIP_SYMBOL(fa::m16::fa_phase_clocks), h.size() * 8));
  double pro = 0, loop = 0, tail = 0, bar = 0, steps = 0, cyc = 0, rt = 0;
  int nw = 0;
  unsigned long long r_first = ~0ull, r_last_start = 0, r_first_end = ~0ull, r_last_end = 0;
  for (int b = 0; b < nwg; ++b) {
    for (int w = 0; w < s.waves; ++w) {
      const unsigned long long* c = &h[(static_cast<size_t>(b) * 16 + w) * 8];
      if (c[0] == 0 || c[3] < c[0]) continue;
      ++nw;
      pro += c[1] - c[0];
      loop += c[2] - c[1];
      tail += c[3] - c[2];
      bar += c[4];
      steps += static_cast<double>(c[7] & 0xffffffffull);
      cyc += c[3] - c[0];
      rt += c[6] - c[5];
      r_first = std::min(r_first, c[5]);
      r_last_start = std::max(r_last_start, c[5]);
      r_first_end = std::min(r_first_end, c[6]);
      r_last_end = std::max(r_last_end, c[6]);
    }
  }
  if (nw == 0) {
    std::printf("%s: no stamps recorded\n", s.name);
    return;
  }
  const double flops = 4.0 * s.B * s.H * static_cast<double>(s.N) * s.N * s.D / (s.causal ? 2 : 1);
  std::printf("%s (B%d H%d N%d D%d %s%s, BR %d x BC %d, %d workgroups x %d waves, %d input sets):\n",
              s.name, s.B, s.H, s.N, s.D, s.bf16 ? "bf16" : "fp16", s.causal ? " causal" : "", s.br,
              s.bc, nwg, s.waves, kSets);
  std::printf("  launch (back to back, %d launches): %.2f us, %.1f TFLOP/s = %.1f %% of 2.5 PFLOP/s\n",
              launches, us, flops / us * 1e-6, flops / us * 1e-6 / 25.0);
  std::printf("  shader clock %.2f GHz; workgroup lifetime %.2f us; span first start -> last end "
              "%.2f us; last start +%.2f us; first end +%.2f us\n",
              cyc / (rt * 10.0), rt / nw * 0.01, (r_last_end - r_first) * 0.01,
              (r_last_start - r_first) * 0.01, (r_first_end - r_first) * 0.01);
  std::printf("  per wave (cycles): prologue %.0f | key walk %.0f = %.1f steps x %.0f "
              "(barrier wait %.0f per step) | merge + epilogue %.0f | total %.0f\n",
              pro / nw, loop / nw, steps / nw, loop / steps, bar / steps, tail / nw, cyc / nw);
  // Per XCD (hardware XCC_ID of wave 0 of each workgroup): how many workgroups ran there, whether
  // workgroup i ran on XCD i % 8 (the grid remap assumes it), and when they started and ended
  // (us after the first start), with the mean lifetime and shader clock.
  int mismatch = 0;
  std::printf("  per XCD: wgs | start first/last | end first/mean/last | lifetime mean | clock\n");
  for (int xcd = 0; xcd < 8; ++xcd) {
    int n = 0;
    double life = 0, endsum = 0, cycs = 0, rts = 0;
    unsigned long long s0 = ~0ull, s1 = 0, e0 = ~0ull, e1 = 0;
    for (int b = 0; b < nwg; ++b) {
      const unsigned long long* c = &h[static_cast<size_t>(b) * 16 * 8];
      if (c[0] == 0 || c[3] < c[0]) continue;
      const int hx = static_cast<int>((c[7] >> 32) & 15u);
      if (xcd == 0 && hx != b % 8) ++mismatch;
      if (hx != xcd) continue;
      ++n;
      life += c[6] - c[5];
      endsum += c[6] - r_first;
      cycs += c[3] - c[0];
      rts += c[6] - c[5];
      s0 = std::min(s0, c[5]);
      s1 = std::max(s1, c[5]);
      e0 = std::min(e0, c[6]);
      e1 = std::max(e1, c[6]);
    }
    if (n == 0) continue;
    std::printf("    XCD %d: %4d | +%.2f / +%.2f | +%.2f / +%.2f / +%.2f | %.2f us | %.2f GHz\n", xcd,
                n, (s0 - r_first) * 0.01, (s1 - r_first) * 0.01, (e0 - r_first) * 0.01,
                endsum / n * 0.01, (e1 - r_first) * 0.01, life / n * 0.01, cycs / (rts * 10.0));
  }
  std::printf("  workgroups not on XCD (index %% 8): %d of %d\n", mismatch, nwg);
  // With PHASE_CLOCKS_DUMP=<dir>, one CSV row per workgroup (wave 0): index, XCC, HW_ID and the
  // s_memrealtime start and end, for offline study of where the dispatcher placed each workgroup.
  if (const char* dir = std::getenv("PHASE_CLOCKS_DUMP")) {
    const std::string path = std::string(dir) + "/" + s.name + ".csv";
    if (FILE* f = std::fopen(path.c_str(), "w")) {
      std::fprintf(f, "bid,xcc,hw_id,start,end\n");
      for (int b = 0; b < nwg; ++b) {
        const unsigned long long* c = &h[static_cast<size_t>(b) * 16 * 8];
        if (c[0] == 0) continue;
        std::fprintf(f, "%d,%llu,%llu,%llu,%llu\n", b, (c[7] >> 32) & 15u, c[7] >> 40,
                     c[5] - r_first, c[6] - r_first);
      }
      std::fclose(f);
    }
  }
  for (int i = 0; i < kSets; ++i) {
    for (void* p : {q[i], k[i], v[i], o[i]}) CHECK(hipFree(p));
    CHECK(hipFree(lse[i]));
  }
  CHECK(hipStreamDestroy(st));
}

}  // namespace

int main(int argc, char** argv) {
  const std::string which = argc > 1 ? argv[1] : "all";
  const int launches = argc > 2 ? std::max(1, std::atoi(argv[2])) : 200;
  bool any = false;
  for (const Shape& s : kShapes) {
    if (which == "all" || which == s.name) {
      run(s, launches);
      any = true;
    }
  }
  if (!any) {
    std::fprintf(stderr, "usage: phase_clocks [C64|C128|C128_causal|LONG|GPT_attn|all] [launches]\n");
    return 2;
  }
  return 0;
}
