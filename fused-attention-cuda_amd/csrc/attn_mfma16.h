// attn_mfma16.h -- the gfx950 fused SDPA forward for 16-bit operands (fp16 / bf16), stages 5 and 4.
//
// Included by attn_f16.hip and attn_bf16.hip. Kernel entry points (profiler-visible names):
//   fa_s5_tuned<T, D, RG, KS, BCW>  stage 5: K/V tiles double-buffered in LDS; the next tile's
//                                   global loads are issued into registers before the current
//                                   tile's math (the reference's PREFETCH, ref:src/stage5_tuned.cu:29-47)
//   fa_s4_mfma<T, D, RG, KS, BCW>   stage 4: the same kernel with one LDS buffer and synchronous
//                                   staging (load -> barrier -> math -> barrier), the reference's
//                                   S4 = S5 with PREFETCH off (ref:src/stage5_tuned.cu:1-8)
//
// Algorithm: FlashAttention-2 loop order with the reference's online-softmax recurrence
// (ref:include/fa/softmax_math.cuh:25-71, ref:src/stage5_tuned.cu:450-726).
//
// Work decomposition (a workgroup = RG*KS waves):
//   * the workgroup owns BR = 32*RG query rows of one (b, h); wave w serves row group rg = w % RG
//     (32 rows) and key split ks = w / RG;
//   * K/V tiles of BC = KS*BCW keys stream through LDS; inside every tile, key split ks takes keys
//     [ks*BCW, (ks+1)*BCW). Each wave therefore runs an independent online softmax over 1/KS of
//     the keys of its rows, and the KS partial states (m, l, O) are merged through LDS at the end.
//   * why split keys: at the canonical size (B2 H8 N2048) there are only 32768 query rows, i.e.
//     32 rows per SIMD on a 256-CU part. With 32-row waves and no split that is one wave per SIMD,
//     and nothing can hide MFMA, exp and LDS latency. With KS = 2 and RG = 4 the workgroup is 8
//     waves (2 per SIMD, 256 workgroups = one per CU) and the two waves of a SIMD interleave.
//
// Per wave and tile (MFMA v_mfma_f32_32x32x16_{f16,bf16}, fp32 accumulate):
//   S^T = K Q^T:  A = K rows from LDS (one 16-byte ds_read_b128 per lane), B = Q from registers.
//                 The 32x32 accumulator gives lane l the query row n = l % 32 and 16 keys
//                 m = 8(r/4) + 4(l/32) + r%4 (r = register), so a row's max/sum needs one
//                 cross-lane step (l ^ 32) and its probabilities are already laid out as the
//                 B operand of the second product.
//   O^T += V^T P^T: A = V^T. V stays row-major in LDS and the operand is read with the gfx950
//                 LDS transpose load ds_read_b64_tr_b16: within each 16-lane group, lane L
//                 receives element L % 4 of the 8 bytes addressed by lanes 4j + L/4 (j = 0..3),
//                 i.e. one head-dim column across 4 keys. Two such reads give the 8 keys
//                 (16h + 8c + 4g + j, c = 0..1, g = l/32) that the probability registers of lane l
//                 hold. P never leaves registers and no VALU transposition is needed.
//
// LDS layout per buffer: Ks[BC][D + 8] then Vs[BC][D + 16] (16-bit elements). The K pad (16 B)
// puts the 8 rows read by 8 consecutive lanes on 8 distinct 16-byte bank groups; the V pad (32 B)
// puts the 4 rows of a 16-lane transpose read on 4 distinct 32-byte bank groups. Tile stores are
// whole 16-byte row segments (conflict-free).
//
// Grid: 1-D, (ceil(N/BR) * B * H) workgroups. Hardware hands workgroup i to XCD i % 8 (each XCD
// has its own L2); blockIdx is remapped so that each XCD receives a contiguous range of
// (head, q-tile) pairs and a head's K/V is fetched into one L2. Causal problems issue the longest
// key ranges first. Causal key tiles past the workgroup's last row are never loaded; per wave,
// 32-key blocks past the wave's last row are skipped and only the diagonal block is masked.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "fa_internal.h"

namespace fa {
namespace m16 {

using ::fa::KArgs;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef s16x4 __attribute__((address_space(3))) lds_s16x4;

constexpr int kNumXcd = 8;
constexpr float kLn2 = 0.69314718055994531f;

// Lazy rescaling threshold in exp2 units: probabilities may reach 2^8 before the running max m is
// moved. bf16 uses 0 (exact running max): with 8 significant bits the largest probability must be
// exactly 1.0, or its own rounding (2^-9 relative) dominates the error of concentrated rows.
template <typename T>
constexpr float lazy_log2() {
  return __is_same(T, __bf16) ? 0.0f : 8.0f;
}

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float log2_hw(float x) { return __builtin_amdgcn_logf(x); }

// 8 fp32 probabilities -> one 16-byte MFMA operand (round to nearest even).
template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* p) {
  if constexpr (__is_same(T, _Float16)) {
    f16x8 h = {(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3],
               (_Float16)p[4], (_Float16)p[5], (_Float16)p[6], (_Float16)p[7]};
    return __builtin_bit_cast(u32x4, h);
  } else {
    bf16x8 h = {(__bf16)p[0], (__bf16)p[1], (__bf16)p[2], (__bf16)p[3],
                (__bf16)p[4], (__bf16)p[5], (__bf16)p[6], (__bf16)p[7]};
    return __builtin_bit_cast(u32x4, h);
  }
}

// acc + the sum of the 8 fp16 values packed in v (4 x v_dot2c_f32_f16 against (1, 1)).
__device__ __forceinline__ float dot2_ones_f16(u32x4 v, float acc) {
  const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
  const f16x8 h = __builtin_bit_cast(f16x8, v);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 0, 1), one, acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 2, 3), one, acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 4, 5), one, acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 6, 7), one, acc, false);
  return acc;
}

template <typename T>
__device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (__is_same(T, _Float16)) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
}

// 8 bytes = four 16-bit elements from LDS through the transpose path (see header).
__device__ __forceinline__ u32x2 lds_read_tr(const void* p) {
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

// T: fp16 or bf16. RG: 32-row groups per workgroup. KS: key splits. BCW: keys per wave per tile.
template <typename T, int D_, int RG, int KS, int BCW, bool PREFETCH>
struct Fa16 {
  static constexpr int D = D_;
  static constexpr int kWaves = RG * KS;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kBr = 32 * RG;
  static constexpr int BC = KS * BCW;
  static constexpr int kLdK = D + 8;   // Ks row stride (elements)
  static constexpr int kLdV = D + 16;  // Vs row stride (elements)
  static constexpr int kKElems = BC * kLdK;
  static constexpr int kBufElems = kKElems + BC * kLdV;
  static constexpr int kBufs = PREFETCH ? 2 : 1;
  static constexpr size_t kTileBytes = static_cast<size_t>(kBufs) * kBufElems * 2;
  static constexpr int kKB = BCW / 32;  // 32-key blocks per wave and tile
  static constexpr int kDB = D / 32;    // 32-wide head-dim blocks of O^T
  static constexpr int kRowChunks = D / 8;           // 16-byte chunks per K/V row
  static constexpr int kChunks = BC * kRowChunks;    // per tensor and tile
  static constexpr int kNC = (kChunks + kThreads - 1) / kThreads;
  // Merge scratch: every non-leading key split writes its O^T registers, m and l per lane.
  static constexpr int kMergeFloats = (kDB * 16 + 2) * 64;
  static constexpr size_t kMergeBytes =
      KS > 1 ? static_cast<size_t>(KS - 1) * RG * kMergeFloats * sizeof(float) : 0;
  static constexpr size_t kLdsBytes = kTileBytes > kMergeBytes ? kTileBytes : kMergeBytes;

  static_assert(BCW % 32 == 0 && BCW >= 32 && BCW <= 128, "BCW must be 32, 64 or 128");
  static_assert(D == 64 || D == 128, "D must be 64 or 128");
  static_assert(kWaves >= 1 && kWaves <= 16, "1..16 waves");
  static_assert(kLdsBytes <= 160 * 1024, "gfx950 LDS is 160 KiB per workgroup");

  struct Staging {
    u32x4 k[kNC];
    u32x4 v[kNC];
  };

  // Global loads of the K/V tile starting at key k0 into registers: thread tid takes 16-byte
  // chunks tid, tid + kThreads, ... (16 consecutive threads read one whole 256-byte row at D=128).
  // Rows past the last key (a partial last tile) are clamped to row N-1: every address stays in
  // the tensor, and those rows sit in 32-key blocks that the math skips.
  __device__ static void load_tile(Staging& st, const T* kb, const T* vb, int k0, int N, int tid) {
    const int last = N - 1 - k0;
#pragma unroll
    for (int i = 0; i < kNC; ++i) {
      const int c = tid + i * kThreads;
      if ((kChunks % kThreads == 0) || c < kChunks) {
        const int row = min(c / kRowChunks, last);
        const size_t off = static_cast<size_t>(k0 + row) * D + (c % kRowChunks) * 8;
        st.k[i] = *reinterpret_cast<const u32x4*>(kb + off);
        st.v[i] = *reinterpret_cast<const u32x4*>(vb + off);
      }
    }
  }

  __device__ static void store_tile(const Staging& st, T* buf, int tid) {
    T* Ks = buf;
    T* Vs = buf + kKElems;
#pragma unroll
    for (int i = 0; i < kNC; ++i) {
      const int c = tid + i * kThreads;
      if ((kChunks % kThreads == 0) || c < kChunks) {
        const int row = c / kRowChunks;
        const int col = (c % kRowChunks) * 8;
        *reinterpret_cast<u32x4*>(Ks + row * kLdK + col) = st.k[i];
        *reinterpret_cast<u32x4*>(Vs + row * kLdV + col) = st.v[i];
      }
    }
  }

  struct WaveState {
    u32x4 q[D / 16];  // B operand of S^T: row n = l%32, head-dim 16*st + 8*(l/32) .. +7
    f32x16 o[kDB];    // O^T accumulator: head-dim rows, query-row columns
    float m;          // running row max (raw score units); may lag the true max (lazy)
    float mc;         // m * c, with 0 while m == -inf
    float l;          // this lane's partial row sum relative to m (the lane pair l, l^32 adds up)
  };

  // One tile for one wave: keys [kbase, kbase + 32*nvalid) of the tile take part; `diag` is the
  // index of the 32-key block on the causal diagonal (-1 if none). vt_lane is the lane's fixed
  // offset of the transpose read (row 4*(l/32) + (l%16)/4, column 16*((l/16)%2) + 4*(l%4)).
  __device__ static void compute_tile(WaveState& ws, const T* buf, int kbase, int nvalid,
                                      int diag, float c, float lazy_raw, int lane, int vt_lane) {
    const T* Ks = buf + kbase * kLdK;
    const T* Vs = buf + kKElems + kbase * kLdV + vt_lane;
    const int g = lane >> 5;
    const int r32 = lane & 31;
    f32x16 s[kKB];
    // ---- S^T = K Q^T ----------------------------------------------------------------------------
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      if (kb < nvalid) {
        f32x16 acc = {};
        const T* krow = Ks + (32 * kb + r32) * kLdK + 8 * g;
#pragma unroll
        for (int st = 0; st < D / 16; ++st) {
          acc = mma<T>(*reinterpret_cast<const u32x4*>(krow + 16 * st), ws.q[st], acc);
        }
        s[kb] = acc;
      }
    }
    // ---- causal diagonal block: key 8(r/4) + 4g + r%4 > row r32 is masked --------------------
    if (diag >= 0) {
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb) {
        if (kb == diag) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            if (8 * (r >> 2) + 4 * g + (r & 3) > r32) s[kb][r] = -__builtin_inff();
          }
        }
      }
    }
    // ---- online softmax with lazy rescaling ----------------------------------------------------
    float mx = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      if (kb < nvalid) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // The running max moves only when some row of the wave sees a score more than lazy_log2
    // (exp2 units) above its current m; otherwise p = exp2(s c - m c) <= 2^lazy_log2 and nothing
    // is rescaled. acc, l and lse all refer to the same m, so the result is unchanged. One ballot
    // per tile: a skipped rescale is a scalar branch.
    if (__builtin_amdgcn_ballot_w64(mx > ws.m + lazy_raw) != 0) {
      const float m_new = fmaxf(ws.m, mx);
      // A row with no visible key so far keeps m = -inf; 0 in the exponent keeps every masked
      // p = exp2(-inf) = 0 and alpha = 0 (acc and l are still 0), never NaN.
      const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
      const float alpha = exp2_hw((ws.m - m_use) * c);
      ws.l *= alpha;
#pragma unroll
      for (int db = 0; db < kDB; ++db) ws.o[db] *= alpha;
      ws.m = m_new;
      ws.mc = m_use * c;
    }
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      if (kb < nvalid) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = exp2_hw(__builtin_fmaf(s[kb][r], c, -ws.mc));
      }
    }
    // ---- O^T += V^T P^T and the row sum ----------------------------------------------------------
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      if (kb < nvalid) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float p[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) p[i] = s[kb][8 * h + i];
          const u32x4 pf = pack8<T>(p);
          u32x4 a[kDB];
#pragma unroll
          for (int db = 0; db < kDB; ++db) {
            const T* vp = Vs + (32 * kb + 16 * h) * kLdV + 32 * db;
            const u32x2 lo = lds_read_tr(vp);
            const u32x2 hi = lds_read_tr(vp + 8 * kLdV);
            a[db] = u32x4{lo[0], lo[1], hi[0], hi[1]};
            ws.o[db] = mma<T>(a[db], pf, ws.o[db]);
          }
          if constexpr (__is_same(T, _Float16)) {
            // fp16: the row sum is taken over the probabilities exactly as they enter the
            // product (rounded to fp16), two per packed dot2.
            rs = dot2_ones_f16(pf, rs);
          } else {
            // bf16 keeps 8 significant bits: the row sum stays in fp32 (the LSE must hold 1e-3),
            // and on the causal diagonal block -- where the first rows of a sequence have all of
            // their few keys -- P is applied as hi + lo (two bf16 operands, exact to ~2^-16).
#pragma unroll
            for (int i = 0; i < 8; ++i) rs += p[i];
            if (kb == diag) {
              float lo[8];
#pragma unroll
              for (int i = 0; i < 8; ++i) lo[i] = p[i] - static_cast<float>(static_cast<__bf16>(p[i]));
              const u32x4 pl = pack8<T>(lo);
#pragma unroll
              for (int db = 0; db < kDB; ++db) ws.o[db] = mma<T>(a[db], pl, ws.o[db]);
            }
          }
        }
      }
    }
    ws.l += rs;
  }

  __device__ static void run(const KArgs& a) {
    __shared__ __attribute__((aligned(16))) char lds_raw[kLdsBytes];
    T* lds = reinterpret_cast<T*>(lds_raw);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // readfirstlane: the wave index and everything derived from it are provably wave-uniform.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = wave % RG;
    const int ks = wave / RG;
    const int g = lane >> 5;

    // XCD-aware remap of the 1-D grid, then (head, q-tile) decode.
    const int G = gridDim.x;
    const int bid = blockIdx.x;
    const int xcd = bid % kNumXcd;
    const int per = G / kNumXcd;
    const int rem = G % kNumXcd;
    const int logical =
        (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + bid / kNumXcd;
    const int bh = logical / a.n_qtiles;
    int qt = logical - bh * a.n_qtiles;
    if (a.causal) qt = a.n_qtiles - 1 - qt;  // longest key ranges first
    const int b = bh / a.H;
    const int h = bh - b * a.H;
    const int hk = h / (a.H / a.Hkv);
    const int N = a.N;

    const size_t q_off = (static_cast<size_t>(b) * a.H + h) * static_cast<size_t>(N) * D;
    const size_t kv_off = (static_cast<size_t>(b) * a.Hkv + hk) * static_cast<size_t>(N) * D;
    const T* qb = static_cast<const T*>(a.q) + q_off;
    const T* kb = static_cast<const T*>(a.k) + kv_off;
    const T* vb = static_cast<const T*>(a.v) + kv_off;

    const int i0 = qt * kBr;
    const int r0 = i0 + 32 * rg;  // this wave's first row
    const bool wave_valid = r0 < N;
    const int row = r0 + (lane & 31);
    // Key range of the workgroup (causal stops at its last row) and of this wave.
    const int kv_end = a.causal ? min(N, i0 + kBr) : N;
    const int n_tiles = (kv_end + BC - 1) / BC;
    const int wave_end = wave_valid ? (a.causal ? min(N, r0 + 32) : N) : 0;

    WaveState ws;
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
      ws.q[st] = wave_valid ? *reinterpret_cast<const u32x4*>(qb + static_cast<size_t>(row) * D +
                                                             16 * st + 8 * g)
                            : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int db = 0; db < kDB; ++db) ws.o[db] = f32x16{};
    ws.m = -__builtin_inff();
    ws.mc = 0.f;
    ws.l = 0.f;

    const int vt_lane = (4 * g + ((lane & 15) >> 2)) * kLdV + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const float lazy_raw = lazy_log2<T>() / a.c;
    const int kbase = ks * BCW;  // this wave's keys inside every tile

    Staging st;
    if constexpr (PREFETCH) {
      load_tile(st, kb, vb, 0, N, tid);
      store_tile(st, lds, tid);
      __syncthreads();
      for (int t = 0; t < n_tiles; ++t) {
        const int k0 = t * BC;
        if (t + 1 < n_tiles) load_tile(st, kb, vb, k0 + BC, N, tid);
        const int kw = k0 + kbase;
        const int nvalid = max(0, min(kKB, (wave_end - kw + 31) / 32));
        if (nvalid > 0) {
          const int diag = a.causal ? (r0 - kw) / 32 : -1;  // r0, kw multiples of 32
          compute_tile(ws, lds + (t & 1) * kBufElems, kbase, nvalid,
                       (diag >= 0 && diag < nvalid) ? diag : -1, a.c, lazy_raw, lane, vt_lane);
        }
        if (t + 1 < n_tiles) store_tile(st, lds + ((t + 1) & 1) * kBufElems, tid);
        __syncthreads();
      }
    } else {
      for (int t = 0; t < n_tiles; ++t) {
        const int k0 = t * BC;
        load_tile(st, kb, vb, k0, N, tid);
        store_tile(st, lds, tid);
        __syncthreads();
        const int kw = k0 + kbase;
        const int nvalid = max(0, min(kKB, (wave_end - kw + 31) / 32));
        if (nvalid > 0) {
          const int diag = a.causal ? (r0 - kw) / 32 : -1;
          compute_tile(ws, lds, kbase, nvalid, (diag >= 0 && diag < nvalid) ? diag : -1, a.c,
                       lazy_raw, lane, vt_lane);
        }
        __syncthreads();
      }
    }

    // ---- merge the KS partial states of each row group (LDS is free after the last barrier) ----
    if constexpr (KS > 1) {
      float* mg = reinterpret_cast<float*>(lds_raw);
      if (ks > 0) {
        float* dst = mg + ((ks - 1) * RG + rg) * kMergeFloats;
#pragma unroll
        for (int db = 0; db < kDB; ++db) {
#pragma unroll
          for (int r = 0; r < 16; ++r) dst[(db * 16 + r) * 64 + lane] = ws.o[db][r];
        }
        dst[kDB * 16 * 64 + lane] = ws.m;
        dst[(kDB * 16 + 1) * 64 + lane] = ws.l;
      }
      __syncthreads();
      if (ks > 0) return;
#pragma unroll
      for (int s = 1; s < KS; ++s) {
        const float* src = mg + ((s - 1) * RG + rg) * kMergeFloats;
        const float m1 = src[kDB * 16 * 64 + lane];
        const float l1 = src[(kDB * 16 + 1) * 64 + lane];
        const float m_new = fmaxf(ws.m, m1);
        const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
        const float a0 = exp2_hw((ws.m - m_use) * a.c);
        const float a1 = exp2_hw((m1 - m_use) * a.c);
        ws.l = ws.l * a0 + l1 * a1;
#pragma unroll
        for (int db = 0; db < kDB; ++db) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            ws.o[db][r] = ws.o[db][r] * a0 + src[(db * 16 + r) * 64 + lane] * a1;
          }
        }
        ws.m = m_new;
      }
    }

    // ---- epilogue: O = acc / l, lse = m*scale + ln l (ref:include/fa/softmax_math.cuh:58-71) ----
    const float lt = ws.l + __shfl_xor(ws.l, 32);
    if (!wave_valid) return;
    const float inv = (lt > 0.f) ? 1.f / lt : 0.f;
    T* orow = static_cast<T*>(a.o) + q_off + static_cast<size_t>(row) * D;
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * db + 8 * j + 4 * g;
        const float x0 = ws.o[db][4 * j + 0] * inv, x1 = ws.o[db][4 * j + 1] * inv;
        const float x2 = ws.o[db][4 * j + 2] * inv, x3 = ws.o[db][4 * j + 3] * inv;
        if constexpr (__is_same(T, _Float16)) {
          *reinterpret_cast<f16x4*>(orow + d) =
              f16x4{(_Float16)x0, (_Float16)x1, (_Float16)x2, (_Float16)x3};
        } else {
          *reinterpret_cast<bf16x4*>(orow + d) =
              bf16x4{(__bf16)x0, (__bf16)x1, (__bf16)x2, (__bf16)x3};
        }
      }
    }
    if (g == 0) {
      a.lse[(static_cast<size_t>(b) * a.H + h) * static_cast<size_t>(N) + row] =
          (lt > 0.f && ws.m != -__builtin_inff()) ? ws.m * a.scale + log2_hw(lt) * kLn2
                                                   : __builtin_inff();
    }
  }
};

template <typename T, int D, int RG, int KS, int BCW>
__global__ __launch_bounds__(64 * RG * KS) void fa_s5_tuned(KArgs a) {
  Fa16<T, D, RG, KS, BCW, true>::run(a);
}

template <typename T, int D, int RG, int KS, int BCW>
__global__ __launch_bounds__(64 * RG * KS) void fa_s4_mfma(KArgs a) {
  Fa16<T, D, RG, KS, BCW, false>::run(a);
}

// Host-side launch of one instantiated variant (STAGE 5 or 4).
template <int STAGE, typename T, int D, int RG, int KS, int BCW>
int launch(const KArgs& in, hipStream_t stream) {
  using A = Fa16<T, D, RG, KS, BCW, STAGE == 5>;
  KArgs a = in;
  a.n_qtiles = (a.N + A::kBr - 1) / A::kBr;
  const long long grid = static_cast<long long>(a.n_qtiles) * a.B * a.H;
  if (grid <= 0 || grid > 0x7fffffffLL) return static_cast<int>(hipErrorInvalidValue);
  const dim3 gr(static_cast<unsigned>(grid)), bl(A::kThreads);
  if constexpr (STAGE == 5) {
    hipLaunchKernelGGL((fa_s5_tuned<T, D, RG, KS, BCW>), gr, bl, 0, stream, a);
  } else {
    hipLaunchKernelGGL((fa_s4_mfma<T, D, RG, KS, BCW>), gr, bl, 0, stream, a);
  }
  return static_cast<int>(hipGetLastError());
}

template <int STAGE, typename T, int D, int RG, int KS, int BCW>
constexpr Variant variant() {
  return Variant{D, 32 * RG, KS * BCW, &launch<STAGE, T, D, RG, KS, BCW>};
}

// ---- instantiation tables: one (RG, KS, BCW) per (BR, BC) -------------------------------------
// Stage 5 rows cover the default tiles, the sweep set and the tile-invariance set, including
// key-split variants at every height so the merge path is tested at small N.
template <typename T, int D>
struct S5Rows {
  static constexpr Variant rows[] = {
      variant<5, T, D, 1, 1, 32>(),   // BR  32, BC  32
      variant<5, T, D, 1, 2, 32>(),   // BR  32, BC  64 (2-way split)
      variant<5, T, D, 2, 1, 32>(),   // BR  64, BC  32
      variant<5, T, D, 2, 2, 32>(),   // BR  64, BC  64 (2-way split)
      variant<5, T, D, 2, 2, 64>(),   // BR  64, BC 128 (2-way split)
      variant<5, T, D, 4, 1, 32>(),   // BR 128, BC  32
      variant<5, T, D, 4, 2, 32>(),   // BR 128, BC  64 (2-way split)
      variant<5, T, D, 4, 2, 64>(),   // BR 128, BC 128 (2-way split) -- default
      variant<5, T, D, 8, 1, 64>(),   // BR 256, BC  64
      variant<5, T, D, 8, 1, 128>(),  // BR 256, BC 128
  };
};

template <typename T>
VariantList s5_table() {
  static const Variant t[] = {
      S5Rows<T, 64>::rows[0],  S5Rows<T, 64>::rows[1],  S5Rows<T, 64>::rows[2],
      S5Rows<T, 64>::rows[3],  S5Rows<T, 64>::rows[4],  S5Rows<T, 64>::rows[5],
      S5Rows<T, 64>::rows[6],  S5Rows<T, 64>::rows[7],  S5Rows<T, 64>::rows[8],
      S5Rows<T, 64>::rows[9],  S5Rows<T, 128>::rows[0], S5Rows<T, 128>::rows[1],
      S5Rows<T, 128>::rows[2], S5Rows<T, 128>::rows[3], S5Rows<T, 128>::rows[4],
      S5Rows<T, 128>::rows[5], S5Rows<T, 128>::rows[6], S5Rows<T, 128>::rows[7],
      S5Rows<T, 128>::rows[8], S5Rows<T, 128>::rows[9]};
  return VariantList{t, static_cast<int>(sizeof(t) / sizeof(t[0]))};
}

// Stage 4: BR fixed at 128 (4 row groups x 2 key splits), BC in {64, 128}; BC 32 without split.
template <typename T>
VariantList s4_table() {
  static const Variant t[] = {variant<4, T, 64, 4, 1, 32>(),  variant<4, T, 64, 4, 2, 32>(),
                              variant<4, T, 64, 4, 2, 64>(),  variant<4, T, 128, 4, 1, 32>(),
                              variant<4, T, 128, 4, 2, 32>(), variant<4, T, 128, 4, 2, 64>()};
  return VariantList{t, static_cast<int>(sizeof(t) / sizeof(t[0]))};
}

}  // namespace m16
}  // namespace fa
