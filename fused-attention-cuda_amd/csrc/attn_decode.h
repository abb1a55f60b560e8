// attn_decode.h -- split-KV decode (flash-decoding) for 16-bit operands on gfx950: Nq new query
// tokens per sequence attend to Nkv cached keys, with the key range cut into splits that run in
// parallel, each writing a partial (O, LSE); a second kernel combines the splits with LSE weights.
// The reference lists this as its next component (ref:README.md:1357-1358) and emits LSE for it
// (ref:include/fa/softmax_math.cuh:65-68); the algorithm is the one its research notes give
// (ref:docs/RESEARCH.md:151-156): O = sum_s e^(L_s - L*) O_s / sum_s e^(L_s - L*), L* = max_s L_s.
//
// Included by attn_f16.hip and attn_bf16.hip. Kernel entry points:
//   fa_decode_split<T, D, RG>  one workgroup per (split, kv head, batch); 4 * RG waves
//   fa_decode_combine<T, D>    one wave per (batch, head, query token)
//
// Work decomposition. The G = H / Hkv query heads of one kv head, times the Nq query tokens, are
// R = G * Nq rows that read the same keys; in q ([B, H, Nq, D]) they are contiguous (head-major,
// then token), so they form RG = 1 or 2 32-row MFMA tiles (R <= 64 is required; rows past R are
// zero). Keys stream through LDS in tiles of 128 (LDS-DMA, two buffers, the next tile in flight
// while the current one is used), shared by the row groups; wave w serves row group w % RG and
// takes keys [32 k, 32 k + 32), k = w / RG, of every tile, and each row group's four partial
// (m, l, O) are merged through LDS at the end (the stage-5 machinery with KS = 4).
// Masking is per lane: row r is query token i = r % Nq, which sees keys j <= Nkv - Nq + i when
// causal (bottom-right: the new tokens are the last Nq positions) and j <= Nkv - 1 otherwise.
// Split boundaries are multiples of 128 keys, so only the last split has a ragged end.
//
// The kernel is bound by HBM reads of K and V (2 Nkv D bytes per element type and kv head).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "attn_mfma16.h"
#include "fa_internal.h"

namespace fa {
namespace m16 {

// One LDS-DMA wave instruction issued as inline asm: lane i copies 16 bytes from `src` to LDS
// byte offset lds + 16 i. Hidden from the compiler, the DMA of the next tile does not make the
// LDS reads of the current tile wait for it (the builtin form would put a vmcnt(0) in front of
// them); the kernel waits itself (vmcnt(0) before the barrier that publishes the tile). M0 is an
// output of the statement, so the compiler knows it is overwritten.
__device__ __forceinline__ void dec_dma16(const void* src, uint32_t lds) {
  uint32_t m0;
  asm volatile("s_mov_b32 %0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               : "={m0}"(m0)
               : "v"(src), "s"(lds)
               : "memory");
}

// RG row groups of 32 query rows (R <= 32 * RG) x 4 key-split waves of 32 keys, 2 buffers.
template <typename T, int D, int RG>
struct Dec16 {
  using F = Fa16<T, D, RG, 4, 32, true>;
  // The decode's LDS: F's double-buffered K/V tiles, reused for the key-split merge at the end.
  // (F's own kLdsBytes also counts the Q region of the forward's prologue, which the decode, with
  // its query rows in registers, does not have.)
  // Merge scratch: each key split's wave writes the three slices of its O^T registers that the
  // other splits finish (kGroups - kOwn groups of 4 registers, 1 KiB each), then m and l per lane.
  static constexpr int kGroups = F::kDB * 4;
  static constexpr int kOwn = kGroups / 4;
  static constexpr size_t kPartBytes = static_cast<size_t>(4) * RG * (kGroups - kOwn) * 64 * 16;
  static constexpr size_t kMergeBytes = kPartBytes + static_cast<size_t>(4) * RG * 64 * 8;
  static constexpr size_t kLdsBytes = F::kTileBytes > kMergeBytes ? F::kTileBytes : kMergeBytes;
  static constexpr int BC = F::BC;        // 128 keys per tile
  static constexpr int kWaves = F::kWaves;
  static constexpr int kThreads = F::kThreads;
  static constexpr int kKB = F::kKB;  // 1
  static constexpr int kDB = F::kDB;

  // The tile of keys [k0, k0 + BC) of one tensor into `buf` through dec_dma16; rows past the
  // range read its last row (N - 1), inside the tensor, and are masked by the math.
  template <bool IS_V>
  __device__ static void dma_tile(T* buf, const T* gbase, const typename F::Dma& d, int k0, int N,
                                  int wave) {
    const T* tile = gbase + static_cast<ptrdiff_t>(k0) * D;
#pragma unroll
    for (int i = 0; i < F::kDmaPerWave; ++i) {
      const int last = min(d.row[i], N - 1 - k0);
      dec_dma16(tile + d.off[i] + (last - d.row[i]) * D,
                static_cast<uint32_t>(reinterpret_cast<uintptr_t>(buf + 512 * (wave + i * kWaves))));
    }
  }

  __device__ static void run(const DecArgs& a) {
    __shared__ __attribute__((aligned(16))) char lds_raw[kLdsBytes];
    T* lds = reinterpret_cast<T*>(lds_raw);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = wave % RG;  // row group: query rows 32 rg .. 32 rg + 31 of the kv head's R
    const int ksp = wave / RG;  // key split: keys 32 ksp .. 32 ksp + 31 of every tile
    const int g = lane >> 5;
    const int s = blockIdx.x % a.S;
    const int bh = blockIdx.x / a.S;
    const int hkv = bh % a.Hkv;
    const int b = bh / a.Hkv;
    const int k_begin = s * a.chunk;
    const int k_end = min(a.Nkv, k_begin + a.chunk);
    const int nk = k_end - k_begin;  // >= 1: the launcher only makes non-empty splits
    const int row = 32 * rg + (lane & 31);
    const bool row_valid = row < a.R;
    const int q0 = (b * a.H + hkv * a.G) * a.Nq;  // first query row of the group in q / o
    const float c = a.c;

    typename F::WaveState ws;
    const T* qrow = static_cast<const T*>(a.q) + static_cast<size_t>(q0 + row) * D;
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
      ws.q[st] = row_valid ? *reinterpret_cast<const u32x4*>(qrow + 16 * st + 8 * g)
                           : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int db = 0; db < kDB; ++db) ws.o[db] = f32x16{};
    ws.m = -__builtin_inff();
    ws.mc = 0.f;
    ws.l = 0.f;
    // Last visible key of this lane's row, relative to k_begin.
    const int tok = row % a.Nq;
    const int lim = (a.causal ? a.Nkv - a.Nq + tok : a.Nkv - 1) - k_begin;
    // bf16 probabilities round to 8 significant bits before the P V MFMA. Over a row's visible
    // keys those rounding errors average out; over a few of them they do not (a flat row over 6
    // keys of unit-variance V errs by up to 2.4e-3). When some row sees fewer than kDecLoKeys keys, every
    // block therefore also carries its probabilities' low parts (P = hi + lo, exact to ~2^-16),
    // as the forward kernel does on its causal diagonal. Wave-uniform; long caches never pay it.
    constexpr int kDecLoKeys = 128;
    const int min_visible = a.causal ? a.Nkv - a.Nq + 1 : a.Nkv;
    const int lo_blk = (!F::kF16 && min_visible < kDecLoKeys) ? 0 : -1;

    const T* kg = static_cast<const T*>(a.k) + static_cast<size_t>(b * a.Hkv + hkv) * a.Nkv * D +
                  static_cast<size_t>(k_begin) * D;
    const T* vg = static_cast<const T*>(a.v) + static_cast<size_t>(b * a.Hkv + hkv) * a.Nkv * D +
                  static_cast<size_t>(k_begin) * D;
    T* const kbuf0 = lds;
    T* const vbuf0 = lds + 2 * F::kKElems;
    const int kbase = ksp * 32;  // this wave's keys inside every tile
    const typename F::KLane kl = F::k_lane(lane);
    const typename F::VLane vl = F::v_lane(lane);
    const typename F::Dma dk = F::template dma_lane<false>(wave, lane, D);
    const typename F::Dma dv = F::template dma_lane<true>(wave, lane, D);
    const int n_tiles = (nk + BC - 1) / BC;

    dma_tile<false>(kbuf0, kg, dk, 0, nk, wave);
    dma_tile<true>(vbuf0, vg, dv, 0, nk, wave);
    F::wait_dma();
    __syncthreads();
    typename F::Probs P;
    f32x16 sc[kKB];
    for (int t = 0; t < n_tiles; ++t) {
      const int buf = t & 1;
      if (t + 1 < n_tiles) {  // the next tile into the other buffer (read in step t-1)
        dma_tile<false>(kbuf0 + (buf ^ 1) * F::kKElems, kg, dk, (t + 1) * BC, nk, wave);
        dma_tile<true>(vbuf0 + (buf ^ 1) * F::kVElems, vg, dv, (t + 1) * BC, nk, wave);
      }
      const int k0 = t * BC + kbase;  // this wave's first key, relative to k_begin
      const int nv = max(0, min(kKB, (nk - k0 + 31) / 32));
      if (nv > 0) {
        const T* ks = kbuf0 + buf * F::kKElems + kbase * D;
        const T* vs = vbuf0 + buf * F::kVElems + kbase * D;
        F::template qk<false>(sc, ws, ks, nv, kl);
        // Per-lane key limit (causal end of the row, or the ragged end of the keys): a select,
        // not a conditional store, so the scores stay in registers.
#pragma unroll
        for (int kb = 0; kb < kKB; ++kb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = k0 + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3);
            sc[kb][r] = key > lim ? -__builtin_inff() : sc[kb][r];
          }
        }
        float mx = 0.f;
        const float rs = F::template softmax_exp<false>(ws, sc, P, mx, nv, -1, c, lane, lo_blk);
        F::template softmax_settle<false>(ws, sc, P, rs, mx, nv, lo_blk, c);
        F::template pv<false>(ws, P, vs, vl, nv, lo_blk);
      }
      F::wait_dma();
      __syncthreads();
    }

    // Merge the four key splits' partial states of each row group (LDS is free after the last
    // barrier), in parallel: the O accumulator's head-dim entries are cut into four slices of
    // kOwn 4-register groups, each split's wave writes the other three slices to LDS, and after
    // one barrier wave ksp merges slice ksp of all four splits: m* = max m_s,
    // w_s = exp2((m_s - m*) c), O = sum_s w_s O_s, l = sum_s w_s l_s, with explicit fused
    // multiply-adds in split order.
    auto group = [&](int gi) __attribute__((always_inline)) {
      return float4{ws.o[gi / 4][4 * (gi % 4) + 0], ws.o[gi / 4][4 * (gi % 4) + 1],
                    ws.o[gi / 4][4 * (gi % 4) + 2], ws.o[gi / 4][4 * (gi % 4) + 3]};
    };
    float4* const parts = reinterpret_cast<float4*>(lds_raw);
    float2* const mls = reinterpret_cast<float2*>(lds_raw + kPartBytes);
    auto part_at = [&](int src, int gi) {  // gi outside src's own slice
      return parts + ((src * RG + rg) * (kGroups - kOwn) + gi - (gi >= src * kOwn ? kOwn : 0)) * 64 +
             lane;
    };
#pragma unroll
    for (int gi = 0; gi < kGroups; ++gi) {
      if (gi / kOwn != ksp) *part_at(ksp, gi) = group(gi);
    }
    mls[(ksp * RG + rg) * 64 + lane] = float2{ws.m, ws.l};
    __syncthreads();
    float ms[4], ls[4];
    float m_fin = -__builtin_inff();
#pragma unroll
    for (int sp = 0; sp < 4; ++sp) {
      const float2 x = mls[(sp * RG + rg) * 64 + lane];
      ms[sp] = x.x;
      ls[sp] = x.y;
      m_fin = fmaxf(m_fin, x.x);
    }
    const float m_use = (m_fin == -__builtin_inff()) ? 0.f : m_fin;
    float lsum = 0.f;
    float4 own[kOwn];
#pragma unroll
    for (int q = 0; q < kOwn; ++q) own[q] = float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sp = 0; sp < 4; ++sp) {
      const float w = exp2_hw((ms[sp] - m_use) * c);
      lsum = __builtin_fmaf(ls[sp], w, lsum);
#pragma unroll
      for (int q = 0; q < kOwn; ++q) {
        float4 x;
        if (sp == ksp) {
          x = group(q);
#pragma unroll
          for (int kk = 1; kk < 4; ++kk) {
            if (ksp == kk) x = group(kk * kOwn + q);
          }
        } else {
          x = *part_at(sp, ksp * kOwn + q);
        }
        own[q] = float4{__builtin_fmaf(x.x, w, own[q].x), __builtin_fmaf(x.y, w, own[q].y),
                        __builtin_fmaf(x.z, w, own[q].z), __builtin_fmaf(x.w, w, own[q].w)};
      }
    }
    const float lt = halves_sum(lsum);
    if (!row_valid) return;
    const bool empty = !(lt > 0.f) || m_fin == -__builtin_inff();
    const float inv = empty ? 0.f : 1.f / lt;
    // lse of the split: m*scale + ln(l); an empty split reports -inf so the combine ignores it,
    // and with a single split the final convention (+inf for a row with no key) applies.
    const float lse = empty ? (a.S == 1 ? __builtin_inff() : -__builtin_inff())
                            : m_fin * a.scale + log2_hw(lt) * kLn2;
    const int d0 = ksp * kOwn * 8;  // first head-dim entry of this wave's slice
    if (a.S == 1) {
      T* orow = static_cast<T*>(a.o) + static_cast<size_t>(q0 + row) * D + d0;
#pragma unroll
      for (int q = 0; q < kOwn; ++q) {
        const float4 x = own[q] * inv;
        if constexpr (F::kF16) {
          *reinterpret_cast<f16x4*>(orow + 8 * q + 4 * g) =
              f16x4{(_Float16)x.x, (_Float16)x.y, (_Float16)x.z, (_Float16)x.w};
        } else {
          *reinterpret_cast<bf16x4*>(orow + 8 * q + 4 * g) =
              bf16x4{(__bf16)x.x, (__bf16)x.y, (__bf16)x.z, (__bf16)x.w};
        }
      }
      if (ksp == 0 && g == 0) a.lse[q0 + row] = lse;
    } else {
      // Partials: o_part [B, Hkv, S, R, D] and lse_part [B, Hkv, S, R], fp32.
      const size_t pr = (static_cast<size_t>(b * a.Hkv + hkv) * a.S + s) * a.R + row;
      float* orow = a.o_part + pr * D + d0;
#pragma unroll
      for (int q = 0; q < kOwn; ++q) {
        *reinterpret_cast<float4*>(orow + 8 * q + 4 * g) = own[q] * inv;
      }
      if (ksp == 0 && g == 0) a.lse_part[pr] = lse;
    }
  }
};

template <typename T, int D, int RG>
__global__ __launch_bounds__(256 * RG) void fa_decode_split(DecArgs a) {
  Dec16<T, D, RG>::run(a);
}

// One wave per output row (b, h, i): the LSE-weighted sum of the S partial rows. Lane l owns
// head-dim elements [D/64 * l, D/64 * (l + 1)). lse = L* + ln(sum_s e^(L_s - L*)); a row whose
// splits are all empty gets O = 0 and lse = +inf (the non-split convention,
// ref:include/fa/softmax_math.cuh:62-68).
// The kernel is a couple of memory round trips per row, so it keeps them few: the splits' LSE are
// read by one lane each (64 splits per load), reduced across the wave, and the partial rows are
// read eight splits per batch of independent loads.
template <typename T, int D>
__global__ __launch_bounds__(256) void fa_decode_combine(DecArgs a) {
  constexpr int kPer = D / 64;
  const int lane = threadIdx.x & 63;
  const int orow = blockIdx.x * 4 + (threadIdx.x >> 6);  // (b, h, i) flattened
  const int n_rows = a.B * a.H * a.Nq;
  if (orow >= n_rows) return;
  const int i = orow % a.Nq;
  const int bh = orow / a.Nq;
  const int h = bh % a.H;
  const int b = bh / a.H;
  const int hkv = h / a.G;
  const int r = (h - hkv * a.G) * a.Nq + i;
  const size_t base = static_cast<size_t>(b * a.Hkv + hkv) * a.S * a.R + r;  // split 0
  const int S = a.S;
  float mx = -__builtin_inff();
  for (int s0 = 0; s0 < S; s0 += 64) {
    const int sl = s0 + lane;
    mx = fmaxf(mx, sl < S ? a.lse_part[base + static_cast<size_t>(sl) * a.R] : -__builtin_inff());
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  float acc[kPer];
#pragma unroll
  for (int e = 0; e < kPer; ++e) acc[e] = 0.f;
  float wsum = 0.f;
  if (mx != -__builtin_inff()) {
    for (int s0 = 0; s0 < S; s0 += 64) {
      const int sl = s0 + lane;
      // This lane's split weight e^(L_s - L*); 0 past S (and for empty splits, L_s = -inf).
      const float wl = sl < S ? __expf(a.lse_part[base + static_cast<size_t>(sl) * a.R] - mx) : 0.f;
      float ws = wl;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) ws += __shfl_xor(ws, off);
      wsum += ws;
      const int n = min(64, S - s0);
      const float* src0 = a.o_part + (base + static_cast<size_t>(s0) * a.R) * D + kPer * lane;
      const size_t step = static_cast<size_t>(a.R) * D;
      int j = 0;
      for (; j + 8 <= n; j += 8) {
        float v[8][kPer];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
#pragma unroll
          for (int e = 0; e < kPer; ++e) v[u][e] = src0[(j + u) * step + e];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float w = __shfl(wl, j + u);
#pragma unroll
          for (int e = 0; e < kPer; ++e) acc[e] += w * v[u][e];
        }
      }
      for (; j < n; ++j) {
        const float w = __shfl(wl, j);
#pragma unroll
        for (int e = 0; e < kPer; ++e) acc[e] += w * src0[j * step + e];
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  T* dst = static_cast<T*>(a.o) + static_cast<size_t>(orow) * D + kPer * lane;
#pragma unroll
  for (int e = 0; e < kPer; ++e) dst[e] = static_cast<T>(acc[e] * inv);
  if (lane == 0) a.lse[orow] = wsum > 0.f ? mx + __logf(wsum) : __builtin_inff();
}

template <typename T, int D>
int launch_decode(const DecArgs& a, hipStream_t stream) {
  const long long grid = static_cast<long long>(a.S) * a.B * a.Hkv;
  if (grid <= 0 || grid > 0x7fffffffLL || a.R < 1 || a.R > 64) {
    return static_cast<int>(hipErrorInvalidValue);
  }
  // One 32-row group for R <= 32; two (8 waves, the same K/V tiles) up to 64 rows.
  if (a.R <= 32) {
    hipLaunchKernelGGL((fa_decode_split<T, D, 1>), dim3(static_cast<unsigned>(grid)),
                       dim3(Dec16<T, D, 1>::kThreads), 0, stream, a);
  } else {
    hipLaunchKernelGGL((fa_decode_split<T, D, 2>), dim3(static_cast<unsigned>(grid)),
                       dim3(Dec16<T, D, 2>::kThreads), 0, stream, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.S == 1) return static_cast<int>(e);
  const long long rows = static_cast<long long>(a.B) * a.H * a.Nq;
  hipLaunchKernelGGL((fa_decode_combine<T, D>), dim3(static_cast<unsigned>((rows + 3) / 4)),
                     dim3(256), 0, stream, a);
  return static_cast<int>(hipGetLastError());
}

}  // namespace m16
}  // namespace fa
