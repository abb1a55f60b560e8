// attn_mfma16.h -- the gfx950 fused SDPA forward for 16-bit operands (fp16 / bf16), stages 5 and 4.
//
// Included by attn_f16.hip and attn_bf16.hip. Kernel entry points (profiler-visible names):
//   fa_s5_tuned<T, D, RG, KS, BCW>  stage 5: software-pipelined. K and V tiles are double-buffered
//                                   in LDS, K one tile ahead of V, and iteration t exponentiates
//                                   tile t while the MFMAs of the next tile's scores run; the
//                                   global loads of later tiles are issued into registers before
//                                   the math (the role of the reference's PREFETCH,
//                                   ref:src/stage5_tuned.cu:29-47)
//   fa_s4_mfma<T, D, RG, KS, BCW>   stage 4: the same math with one LDS buffer and synchronous
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
// LDS layout: K and V tiles are BC rows of D 16-bit elements, unpadded, with the 16-byte chunks
// of each row XOR-swizzled (K by row & 7, V by 2 (row & 3)) so that the 8 rows of one K operand
// read and the 4 rows of one V transpose read hit distinct banks. Tiles are written straight
// from HBM by global_load_lds_dwordx4 (no register staging), one contiguous KiB per wave
// instruction; the swizzle is applied on the global side by choosing each lane's source chunk.
//
// Grid: 1-D, (ceil(N/BR) * B * H) workgroups. Hardware hands workgroup i to XCD (i + c) % 8, c
// fixed for the launch (each XCD has its own L2); blockIdx is remapped so that each XCD receives
// a contiguous range of (head, q-tile) pairs and a head's K/V is fetched into one L2
// (layout::grid_item). Causal problems issue the longest key ranges first, across all heads of an
// XCD's range when that range is whole heads. Causal key tiles past the workgroup's last row are
// never loaded; per wave, 32-key blocks past the wave's last row are skipped and only the diagonal
// block is masked.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <type_traits>

#include "fa_internal.h"
#include "wave_halves.h"
#include "tile_layout.h"

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

constexpr float kLn2 = 0.69314718055994531f;

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// floor(n / d) for 0 <= n < 2^31 from the launch's precomputed FastDiv (two scalar instructions
// for a uniform n).
__device__ __forceinline__ int fdiv(int n, const FastDiv& f) {
  return f.d == 1 ? n : static_cast<int>(__umulhi(static_cast<uint32_t>(n), f.m) >> f.s);
}
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
// PIPE: software-pipelined stage-5 loop (see run()); false = the synchronous stage-4 loop.
template <typename T, int D_, int RG, int KS, int BCW, bool PIPE>
struct Fa16 {
  static constexpr int D = D_;
  static constexpr bool kF16 = __is_same(T, _Float16);
  static constexpr int kWaves = RG * KS;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kBr = 32 * RG;
  static constexpr int BC = KS * BCW;
  static constexpr int kKElems = BC * D;  // one K buffer (unpadded rows, swizzled chunks)
  static constexpr int kVElems = BC * D;  // one V buffer
  static constexpr int kBufs = PIPE ? 2 : 1;
  static constexpr size_t kTileBytes = static_cast<size_t>(kBufs) * (kKElems + kVElems) * 2;
  // Stage 5 stages the workgroup's Q tile through LDS as well (K layout, BR rows): every prologue
  // load is then an LDS-DMA, so the first memory round trip carries Q, K(0), V(0) and K(1) at once
  // and the kernel waits for exactly the loads it needs (see run()).
  static constexpr size_t kQBytes = PIPE ? static_cast<size_t>(kBr) * D * 2 : 0;
  static constexpr int kQInsts = kBr * D / 8 / 64 / kWaves;  // Q LDS-DMA instructions per wave
  static constexpr int kKB = BCW / 32;  // 32-key blocks per wave and tile
  static constexpr int kDB = D / 32;    // 32-wide head-dim blocks of O^T
  static constexpr int kRowChunks = D / 8;         // 16-byte chunks per K/V row
  static constexpr int kChunks = BC * kRowChunks;  // per tensor and tile
  static constexpr int kDmaInsts = kChunks / 64;   // 1 KiB LDS-DMA instructions per tensor/tile
  static constexpr int kDmaPerWave = kDmaInsts / kWaves;
  // Merge and epilogue (run() after the key walk). The O^T accumulator of a wave is kGroups groups
  // of 4 registers; group gi = 4 db + j holds head-dim entries 32 db + 8 j + 4 (lane / 32) + 0..3
  // of the lane's row. The KS waves of a row group split the groups: wave ks finishes the kOwn
  // groups [ks kOwn, (ks + 1) kOwn), a contiguous slice of kSliceD head-dim entries.
  static constexpr int kGroups = kDB * 4;
  static constexpr int kOwn = kGroups / KS;
  static constexpr int kSliceD = kOwn * 8;
  // Merge scratch: every wave writes the groups the other waves finish (KS - 1 slices of 1 KiB per
  // group), then m and l per lane.
  static constexpr size_t kPartBytes =
      static_cast<size_t>(KS - 1) * RG * KS * kOwn * 64 * 16;
  static constexpr size_t kMergeBytes =
      KS > 1 ? kPartBytes + static_cast<size_t>(KS) * RG * 64 * 8 : 0;
  // Output staging: 32 rows of the wave's slice, each padded by 16 bytes.
  static constexpr int kStageRow = kSliceD + 8;  // elements
  static constexpr size_t kStageBytes = static_cast<size_t>(RG) * KS * 32 * kStageRow * 2;
  static constexpr size_t kEpiBytes = kMergeBytes > kStageBytes ? kMergeBytes : kStageBytes;
  static constexpr size_t kLdsBytes =
      kTileBytes + kQBytes > kEpiBytes ? kTileBytes + kQBytes : kEpiBytes;
  // fp16 fast path: p = exp2(s c - m c) is used as long as every probability of the tile stays
  // <= 2^14 (so the fp16 operand, max 65504, cannot overflow); the check is the lane's tile row
  // sum, which bounds each of its probabilities.
  static constexpr float kF16SumLimit = 16384.0f;

  static_assert(BCW % 32 == 0 && BCW >= 32 && BCW <= 128, "BCW must be 32, 64 or 128");
  static_assert(D == 64 || D == 128, "D must be 64 or 128");
  static_assert(kWaves >= 1 && kWaves <= 16, "1..16 waves");
  static_assert(kLdsBytes <= 160 * 1024, "gfx950 LDS is 160 KiB per workgroup");
  static_assert(kChunks % 64 == 0, "a tile is a whole number of 1 KiB DMA instructions");
  static_assert(kDmaInsts % kWaves == 0, "every wave issues the same number of DMA instructions");
  static_assert(kBr * D / 8 % (64 * kWaves) == 0, "the Q tile is whole DMA instructions per wave");
  static_assert(2 * kDmaPerWave < 64, "prologue vmcnt immediates fit 6 bits");
  static_assert(kGroups % KS == 0 && kOwn % 2 == 0, "whole, even slices of O^T groups per wave");
  static_assert(KS == 1 || 32 * kStageRow * 2 <= kOwn * 64 * 16,
                "a wave's staging fits its slice of one other wave's merge scratch");

  // LDS layout of a K/V tile (layout::swz): BC rows of D elements, unpadded, with the 16-byte
  // chunks of each row XOR-swizzled by a function of the row chosen by measured read rate.
  template <bool IS_V>
  __device__ static int swz(int row) {
    return layout::swz<D, IS_V>(row);
  }

  // Tiles go straight from HBM into LDS with global_load_lds_dwordx4: lane i of a wave
  // instruction writes LDS bytes [16 i, 16 i + 16) of that instruction's 1 KiB (M0 + 16 * lane,
  // verified on the box), so the global side picks, per lane, the chunk that belongs at that
  // position. Instruction j of a tile goes to wave j % kWaves. Dma holds a lane's source for each
  // of its instructions relative to the tile's first key: the tile-local row and the element
  // offset row * D + swizzled chunk * 8 (loop-invariant).
  struct Dma {
    int row[kDmaPerWave];
    int off[kDmaPerWave];
  };
  template <bool IS_V>
  __device__ static Dma dma_lane(int wave, int lane, int sn) {
    Dma d;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
      const auto src = layout::dma_src<D, IS_V>(kWaves, wave, lane, i, sn);
      d.row[i] = src.row;
      d.off[i] = src.off;
    }
    return d;
  }

  // The tile of keys [k0, k0 + BC) of one tensor (row stride sn) into `buf`. Rows past the last
  // key (a partial last tile) read row N-1: every address stays in the tensor, and those rows
  // sit in 32-key blocks that the math skips. The caller waits on vmcnt before the barrier that
  // publishes it.
  template <bool IS_V>
  __device__ static void dma_tile(T* buf, const T* gbase, const Dma& d, int k0, int N, int sn,
                                  int wave) {
    const T* tile = gbase + static_cast<ptrdiff_t>(k0) * sn;
    if (k0 + BC <= N) {  // workgroup-uniform
#pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i) {
        __builtin_amdgcn_global_load_lds(
            (const void __attribute__((address_space(1)))*)(tile + d.off[i]),
            (void __attribute__((address_space(3)))*)(buf + 512 * (wave + i * kWaves)), 16, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i) {
        const int last = min(d.row[i], N - 1 - k0);
        __builtin_amdgcn_global_load_lds(
            (const void __attribute__((address_space(1)))*)(tile + d.off[i] + (last - d.row[i]) * sn),
            (void __attribute__((address_space(3)))*)(buf + 512 * (wave + i * kWaves)), 16, 0, 0);
      }
    }
  }

  // dma_tile for a tile known to lie inside the tensor (k0 + BC <= N): no clamp, no branch.
  template <bool IS_V>
  __device__ static void dma_tile_full(T* buf, const T* gbase, const Dma& d, int k0, int sn,
                                       int wave) {
    const T* tile = gbase + static_cast<ptrdiff_t>(k0) * sn;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(tile + d.off[i]),
          (void __attribute__((address_space(3)))*)(buf + 512 * (wave + i * kWaves)), 16, 0, 0);
    }
  }

  // Waits until this wave's LDS-DMA loads have landed (vmcnt(0); expcnt and lgkmcnt untouched).
  __device__ static void wait_dma() { __builtin_amdgcn_s_waitcnt(0x0F70); }
  // Waits until at most n (< 64) of this wave's loads are outstanding: they complete in issue
  // order, so every load issued before the last n has landed. vmcnt is split over bits 3:0 and
  // 15:14 of the immediate.
  template <int n>
  __device__ static void wait_dma_but() {
    static_assert(n >= 0 && n < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (n & 15) | ((n >> 4) << 14));
  }

  // One 1 KiB LDS-DMA instruction from inline assembly. The compiler does not see it as a load
  // that may write LDS, so it adds no vmcnt wait of its own before later LDS reads; the caller
  // waits for it explicitly (wait_dma) before the barrier that publishes the tile.
  __device__ static void dma_asm(const void* src, const void* lds) {
    uint32_t m0;
    asm volatile("s_mov_b32 %0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 : "={m0}"(m0)
                 : "v"(src), "s"(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)))
                 : "memory");
  }
  // dma_tile through dma_asm (rows past the last key read row N-1, as in dma_tile).
  template <bool IS_V>
  __device__ static void dma_tile_asm(T* buf, const T* gbase, const Dma& d, int k0, int N, int sn,
                                      int wave) {
    const T* tile = gbase + static_cast<ptrdiff_t>(k0) * sn;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
      const int last = min(d.row[i], N - 1 - k0);
      dma_asm(tile + d.off[i] + (last - d.row[i]) * sn, buf + 512 * (wave + i * kWaves));
    }
  }

  struct WaveState {
    u32x4 q[D / 16];  // B operand of S^T: row n = l%32, head-dim 16*st + 8*(l/32) .. +7
    f32x16 o[kDB];    // O^T accumulator: head-dim rows, query-row columns
    float m;          // reference max of the row (raw score units); p = exp2(s c - m c)
    float mc;         // m * c, with 0 while m == -inf
    float l;          // this lane's partial row sum relative to m (the lane pair l, l^32 adds up)
  };

  // Probabilities of one tile as MFMA operands: p[kb][h] covers keys 16h..16h+15 of block kb;
  // plo holds the bf16 low parts of the causal diagonal block.
  struct Probs {
    u32x4 p[kKB][2];
    u32x4 plo[2];
  };

  // S^T = K Q^T for the valid 32-key blocks (all of them when FULL). Ks points at the wave's keys.
  // Lane l reads key row l % 32 of each block, chunk 2 st + l / 32 (head-dim 16 st + 8 (l/32));
  // the row's swizzle is swz(l % 32) because every 32-key block starts at a multiple of 32. The
  // lane's offsets are loop-invariant: KLane holds them.
  struct KLane {
    int off[D / 16];
  };
  __device__ static KLane k_lane(int lane) {
    KLane k;
#pragma unroll
    for (int st = 0; st < D / 16; ++st) k.off[st] = layout::k_operand_offset<D>(lane, st);
    return k;
  }
  template <bool FULL>
  __device__ static void qk(f32x16 (&s)[kKB], const WaveState& ws, const T* Ks, int nvalid,
                            const KLane& kl) {
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      if (FULL || kb < nvalid) {
        f32x16 acc = {};
#pragma unroll
        for (int st = 0; st < D / 16; ++st) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(Ks + 32 * kb * D + kl.off[st]);
          acc = mma<T>(a, ws.q[st], acc);
        }
        s[kb] = acc;
      }
    }
  }

  // The row max of a tile: the lane's own 16 (32, 64) scores, then the other half of the row (lane
  // l ^ 32) through halves_max, a VALU exchange of the wave's two 32-lane halves, instead of an
  // LDS bpermute round trip (measured: LONG, bf16, -1.5 to -2 %; bit-identical).
  template <bool FULL>
  __device__ static float tile_max(const f32x16 (&s)[kKB], int nvalid) {
    float mx = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      if (FULL || kb < nvalid) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      }
    }
    return halves_max(mx);
  }

  // Moves the reference max to max(m, mx) and rescales l and O by alpha = exp2((m_old - m_new) c).
  __device__ static void rescale(WaveState& ws, float mx, float c) {
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

  // p = exp2(s c - m c) for the valid blocks, packed into P. Returns this lane's share of the
  // tile's row sum: over the fp16-rounded values (two per packed dot2) for fp16, so numerator and
  // denominator use the same weights; in fp32 for bf16, whose 8 significant bits would cost the
  // LSE its 1e-3. For bf16 the causal diagonal block also gets its low parts (P = hi + lo, exact
  // to ~2^-16): the first rows of a sequence have all of their few keys in that block.
  template <bool FULL>
  __device__ static float exp_pack(const f32x16 (&s)[kKB], Probs& P, const WaveState& ws,
                                   int nvalid, int diag, float c) {
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      if (FULL || kb < nvalid) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float p[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) p[i] = exp2_hw(__builtin_fmaf(s[kb][8 * h + i], c, -ws.mc));
          P.p[kb][h] = pack8<T>(p);
          if constexpr (kF16) {
            rs = dot2_ones_f16(P.p[kb][h], rs);
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) rs += p[i];
            if (!FULL && kb == diag) {
              float lo[8];
#pragma unroll
              for (int i = 0; i < 8; ++i) lo[i] = p[i] - static_cast<float>(static_cast<__bf16>(p[i]));
              P.plo[h] = pack8<T>(lo);
            }
          }
        }
      }
    }
    return rs;
  }

  // Online softmax of one tile (ref:include/fa/softmax_math.cuh:25-71), in two halves.
  // softmax_exp masks the causal diagonal block and exponentiates against the current reference
  // max m; softmax_settle then settles m:
  //   fp16 -- lazy: m stays as long as every probability of the tile is <= 2^14 (the lane's tile
  //           sum bounds each of its probabilities, and fp16 holds 65504) and the row has a
  //           reference; otherwise the wave takes the tile max, rescales and redoes the tile;
  //   bf16 -- exact: m is the running max, so the largest probability is exactly 1.0 (a rounded
  //           largest probability would dominate the error of concentrated rows).
  // acc, l and lse all refer to the same m and m only moves to an observed max, so the result is
  // the reference's recurrence. The decision is one ballot (a scalar branch).
  // `lo` names the block whose bf16 probabilities also get their low parts: the causal diagonal
  // block by default (kLoAtDiag); the decode passes its own choice with diag = -1 (no mask).
  static constexpr int kLoAtDiag = -2;
  template <bool FULL>
  __device__ static float softmax_exp(WaveState& ws, f32x16 (&s)[kKB], Probs& P, float& mx,
                                      int nvalid, int diag, float c, int lane,
                                      int lo = kLoAtDiag) {
    if (!FULL && diag >= 0) {
      const int g = lane >> 5;
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb) {
        if (kb == diag) {
          // A select, not a conditional store: conditional element stores keep the score
          // registers in scratch memory.
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            s[kb][r] = (8 * (r >> 2) + 4 * g + (r & 3) > (lane & 31)) ? -__builtin_inff() : s[kb][r];
          }
        }
      }
    }
    if constexpr (!kF16) mx = tile_max<FULL>(s, nvalid);
    return exp_pack<FULL>(s, P, ws, nvalid, lo == kLoAtDiag ? diag : lo, c);
  }

  template <bool FULL>
  __device__ static void softmax_settle(WaveState& ws, const f32x16 (&s)[kKB], Probs& P, float rs,
                                        float mx, int nvalid, int diag, float c) {
    bool redo;
    if constexpr (kF16) {
      redo = !(rs <= kF16SumLimit) || ws.m == -__builtin_inff();
    } else {
      redo = mx > ws.m;
    }
    if (__builtin_amdgcn_ballot_w64(redo) != 0) {
      if constexpr (kF16) mx = tile_max<FULL>(s, nvalid);
      rescale(ws, mx, c);
      rs = exp_pack<FULL>(s, P, ws, nvalid, diag, c);
    }
    ws.l += rs;
  }

  // V^T operands of one tile: va[kb][h][db] covers keys 32kb + 16h .. +15 and head-dim block db.
  // Vs points at the wave's keys. Lane l = 16 G + 4 j + q of a transpose read addresses key
  // row 4 (G/2) + j (+ 8 for the second read) at head-dim 32 db + 16 (G%2) + 4 q; the row's
  // swizzle is swz(j) (rows start at multiples of 4), so the lane's offset for block db is a
  // loop-invariant per-lane constant, VLane::off[db].
  using VOps = u32x4[kKB][2][kDB];
  struct VLane {
    int off[kDB];
  };
  __device__ static VLane v_lane(int lane) {
    VLane v;
#pragma unroll
    for (int db = 0; db < kDB; ++db) v.off[db] = layout::v_operand_offset<D>(lane, db);
    return v;
  }
  __device__ static u32x4 v_operand(const T* Vs, const VLane& vl, int kb, int h, int db) {
    const T* vp = Vs + (32 * kb + 16 * h) * D + vl.off[db];
    const u32x2 lo = lds_read_tr(vp);
    const u32x2 hi = lds_read_tr(vp + 8 * D);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  }

  // O^T += V^T P^T (operands read here; the partial-tile path).
  template <bool FULL>
  __device__ static void pv(WaveState& ws, const Probs& P, const T* Vs, const VLane& vl, int nvalid,
                            int diag) {
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      if (FULL || kb < nvalid) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int db = 0; db < kDB; ++db) {
            const u32x4 a = v_operand(Vs, vl, kb, h, db);
            ws.o[db] = mma<T>(a, P.p[kb][h], ws.o[db]);
            if constexpr (!kF16) {
              if (!FULL && kb == diag) ws.o[db] = mma<T>(a, P.plo[h], ws.o[db]);
            }
          }
        }
      }
    }
  }

  // The steady-state step on full tiles: S(t+1) = K(t+1) Q^T on MFMA, interleaved with the
  // exponentials of S(t); every LDS read of the step (K rows of t+1 and the V^T operands of t) is
  // issued up front so that no MFMA waits on LDS latency; then the P(t) V(t) MFMAs. `prefetch`
  // issues the LDS-DMA of later tiles after those reads: the compiler cannot tell a DMA's LDS
  // target from the buffers read here and makes any LDS read that follows a DMA wait for it
  // (vmcnt(0)), which would expose the whole memory latency in every step.
  template <typename Prefetch>
  __device__ static void step_full(WaveState& ws, f32x16 (&s_cur)[kKB], f32x16 (&s_nxt)[kKB],
                                   Probs& P, const T* Kn, const T* Vc, const KLane& kl,
                                   const VLane& vl, float c, int lane, Prefetch&& prefetch) {
    VOps va;
    // Wave priority: raised for the first half of the step (LDS reads, DMA, S(t+1) MFMAs with the
    // exponentials of S(t)) and dropped for the settle and the P(t) V(t) MFMAs. A wave that
    // reaches its second half first thus yields issue to its SIMD partner still in the first,
    // instead of the older wave taking every contested slot and the younger one finishing the
    // step alone (measured: C128 44.3 -> 42.1 us, C64 and LONG -0.8 %).
    __builtin_amdgcn_s_setprio(1);
    qk<true>(s_nxt, ws, Kn, kKB, kl);
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int db = 0; db < kDB; ++db) va[kb][h][db] = v_operand(Vc, vl, kb, h, db);
      }
    }
    prefetch();
    float mx = 0.f;
    const float rs = softmax_exp<true>(ws, s_cur, P, mx, kKB, -1, c, lane);
    // Issue order for the region: the K reads, then the V^T reads, then the DMA, then one MFMA of
    // S(t+1) per group of VALU ops. While an MFMA runs in the matrix core the wave keeps issuing
    // independent VALU work (issue is in order, so a cluster of MFMAs would stall it).
    constexpr int kMfma = kKB * (D / 16);
    constexpr int kVReads = kKB * 2 * kDB * 2;
    constexpr int kValu = (kF16 ? 48 : 66) * kKB;
    // VALU ops per MFMA: by default the step's softmax VALU spread evenly over the S(t+1) MFMAs
    // (the rest issue after the last one). Tiles where fewer per MFMA measured faster
    // (same-box A/B, eager launches, bit-identical outputs), against the even spread:
    //   fp16 D64, two 32-key blocks per wave (C64's BR 128 x BC 128): 4 against 12,
    //     C64 -3.4 to -3.9 %, C64 causal at BR 64 -2.7 %;
    //   bf16 D128, one key split (LONG's BR 128 x BC 32): 4 against 9, -1.5 %.
    // C128's tile keeps its 6 (3, 4 and 8 measured 1 to 2 % slower), and the GPT-2 attention
    // shape's D64 tile with one block per wave its 12 (8: median of 12 pairs within 0.3 %).
    constexpr int kPerEven = (kValu + kMfma - 1) / kMfma;
    constexpr int kPer = (kF16 && D == 64 && kKB == 2)    ? 4
                         : (!kF16 && D == 128 && KS == 1) ? 4
                                                          : kPerEven;
    __builtin_amdgcn_sched_group_barrier(0x100, kMfma, 0);    // DS reads: K rows
    __builtin_amdgcn_sched_group_barrier(0x100, kVReads, 0);  // DS reads: V^T operands
    __builtin_amdgcn_sched_group_barrier(0x020, 2 * kDmaPerWave, 0);  // VMEM: the DMA
#pragma unroll
    for (int i = 0; i < kMfma; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x002, kPer, 0);  // VALU
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // MFMA
    }
    __builtin_amdgcn_s_setprio(0);
    softmax_settle<true>(ws, s_cur, P, rs, mx, kKB, -1, c);
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int db = 0; db < kDB; ++db) ws.o[db] = mma<T>(va[kb][h][db], P.p[kb][h], ws.o[db]);
      }
    }
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

    // XCD-aware decode of the 1-D grid into (head, query tile, part). (readfirstlane: uniform
    // integer divisions run on the vector unit, and their results would otherwise occupy vector
    // registers for the whole kernel.)
    const layout::Item item = layout::grid_item(
        static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x), a.n_qtiles, a.n_splits,
        a.causal != 0, a.xcd_heads, a.xcd_cus,
        [&](int x) { return __builtin_amdgcn_readfirstlane(fdiv(x, a.fd_splits)); },
        [&](int x) { return __builtin_amdgcn_readfirstlane(fdiv(x, a.fd_qtiles)); },
        [&](int x) { return __builtin_amdgcn_readfirstlane(fdiv(x, a.fd_xcd_heads)); },
        [&](int x) { return __builtin_amdgcn_readfirstlane(fdiv(x, a.fd_xcd_cus)); });
    const int S = a.n_splits;
    const int part = __builtin_amdgcn_readfirstlane(item.part);
    const int bh = __builtin_amdgcn_readfirstlane(item.bh);
    const int qt = __builtin_amdgcn_readfirstlane(item.qt);
    const int b = fdiv(bh, a.fd_h);
    const int h = bh - b * a.H;
    const int hk = fdiv(h, a.fd_group);
    const int N = a.N;

    const T* qb = static_cast<const T*>(a.q) + b * a.qsb + h * a.qsh;
    const T* kg = static_cast<const T*>(a.k) + b * a.ksb + hk * a.ksh;
    const T* vg = static_cast<const T*>(a.v) + b * a.vsb + hk * a.vsh;

    const int i0 = qt * kBr;
    const int r0 = i0 + 32 * rg;  // this wave's first row
    const bool wave_valid = r0 < N;
    const int row = r0 + (lane & 31);
    // Key range of the workgroup (causal stops at its last row) and of this wave. The workgroup
    // walks key tiles [t0, n_tiles): the whole walk, or its part of a split walk; steps before
    // n_steady take the steady body (layout::plan_walk).
    layout::Walk walk = layout::plan_walk(N, BC, kBr, qt, a.causal != 0, part,
                                          [&](int x) { return fdiv(x, a.fd_splits); });
    if (PIPE && a.rotate) {
      layout::rotate_walk(walk, N, BC, kBr, qt, a.causal != 0, part,
                          [&](int x) { return fdiv(x, a.fd_splits); },
                          [&](int x) { return fdiv(x, a.fd_rot_blocks); }, a.rot_lg);
    }
    walk.rot = __builtin_amdgcn_readfirstlane(walk.rot);
    walk.rot_end = __builtin_amdgcn_readfirstlane(walk.rot_end);
    // Key tile of walk step t (in order, or rotated: layout::walk_tile).
    auto wt = [&](int t) { return layout::walk_tile(walk, t); };
    const int t0 = __builtin_amdgcn_readfirstlane(walk.t0);
    const int n_tiles = __builtin_amdgcn_readfirstlane(walk.n_tiles);
    const int wave_end = wave_valid ? (a.causal ? min(N, r0 + 32) : N) : 0;
    const int kbase = ks * BCW;  // this wave's keys inside every tile
    const float c = a.c;

    WaveState ws;
    if constexpr (!PIPE) {
#pragma unroll
      for (int st = 0; st < D / 16; ++st) {
        ws.q[st] = wave_valid ? *reinterpret_cast<const u32x4*>(qb + row * a.qsn + 16 * st + 8 * g)
                              : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int db = 0; db < kDB; ++db) ws.o[db] = f32x16{};
    ws.m = -__builtin_inff();
    ws.mc = 0.f;
    ws.l = 0.f;

    // Buffers: K[kBufs] then V[kBufs]; the wave's view starts at its key split.
    T* const kbuf0 = lds;
    T* const vbuf0 = lds + kBufs * kKElems;
    const KLane kl = k_lane(lane);
    const VLane vl = v_lane(lane);
    const int ksn = a.ksn, vsn = a.vsn;
    const Dma dk = dma_lane<false>(wave, lane, ksn);
    const Dma dv = dma_lane<true>(wave, lane, vsn);
    auto kwave = [&](int buf) -> const T* { return kbuf0 + buf * kKElems + kbase * D; };
    auto vwave = [&](int buf) -> const T* { return vbuf0 + buf * kVElems + kbase * D; };
    // Valid 32-key blocks of tile t for this wave, and its causal diagonal block (-1 if none).
    auto nvalid_of = [&](int t) -> int {
      return max(0, min(kKB, (wave_end - (t * BC + kbase) + 31) / 32));
    };
    auto diag_of = [&](int t, int nv) -> int {
      const int d = a.causal ? (r0 - (t * BC + kbase)) / 32 : -1;  // multiples of 32
      return (d >= 0 && d < nv) ? d : -1;
    };

    Probs P;
    if constexpr (PIPE) {
     if (t0 < n_tiles) {  // workgroup-uniform: an empty part of a split walk loads nothing
      // Software pipeline: iteration t exponentiates tile t while the MFMAs of S(t+1) = K(t+1) Q^T
      // run, then applies P(t) to V(t). K is therefore staged one tile ahead of V: with u = t - t0,
      // iteration t reads K buffer (u+1)%2 and V buffer u%2 and refills K buffer u%2 with K(t+2)
      // and V buffer (u+1)%2 with V(t+1).
      // Prologue: one memory round trip. Q (into its own LDS region, K layout), K(t0), V(t0) and
      // K(t0+1) are all in flight at once, through inline-asm DMA: the compiler tracks none of
      // them, so it adds no wait of its own, and the kernel waits for exactly what it reads --
      // Q and K(t0) (issued first) before QK(t0), the rest (landing while QK(t0) runs) before the
      // second barrier. Q rows past N read row N-1 (their waves store nothing).
      {
        T* const qbuf = lds + kBufs * (kKElems + kVElems);
        const T* qtile = static_cast<const T*>(a.q) + b * a.qsb + h * a.qsh;
#pragma unroll
        for (int i = 0; i < kQInsts; ++i) {
          const auto src = layout::dma_src<D, false>(kWaves, wave, lane, i, a.qsn);
          const int qrow = min(i0 + src.row, N - 1);
          dma_asm(qtile + src.off + (qrow - src.row) * a.qsn, qbuf + 512 * (wave + i * kWaves));
        }
        dma_tile_asm<false>(kbuf0, kg, dk, wt(t0) * BC, N, ksn, wave);
        dma_tile_asm<true>(vbuf0, vg, dv, wt(t0) * BC, N, vsn, wave);
        if (t0 + 1 < n_tiles) {
          dma_tile_asm<false>(kbuf0 + kKElems, kg, dk, wt(t0 + 1) * BC, N, ksn, wave);
          wait_dma_but<2 * kDmaPerWave>();
        } else {
          wait_dma_but<kDmaPerWave>();
        }
        __syncthreads();  // Q and K(t0) visible
#pragma unroll
        for (int st = 0; st < D / 16; ++st)
          ws.q[st] = *reinterpret_cast<const u32x4*>(qbuf + 32 * rg * D + kl.off[st]);
      }
      f32x16 sa[kKB], sb[kKB];
      {
        const int nv0 = nvalid_of(wt(t0));
        if (nv0 > 0) qk<false>(sa, ws, kwave(0), nv0, kl);
      }
      // When the first step is a steady one (tile t0 full and free of the causal diagonal), the
      // reference max starts at the row max of S(t0), taken here. Otherwise the first step
      // exponentiates against m = -inf, finds no reference and redoes the tile: once per walk,
      // in both precisions. The results are the same: the redo moved m to this max and scaled
      // the still-empty l and O by 0.
      if (__builtin_amdgcn_readfirstlane(walk.n_steady) > t0) {
        const float mx = tile_max<true>(sa, kKB);
        ws.m = mx;
        ws.mc = (mx == -__builtin_inff()) ? 0.f : mx * c;
      }
      wait_dma();
      __syncthreads();  // V(t0), K(t0+1) visible; K buffer 0 is refilled in iteration 0
      // One pipeline step. `full` (a compile-time tag) selects the steady-state body: tiles t and
      // t+1 are full for every wave of the workgroup and carry no causal diagonal, so the body has
      // no per-block branches and the VALU softmax of S(t) interleaves with the MFMAs of S(t+1).
      // The parity tag makes the calls with swapped S arrays distinct instantiations (one function
      // called with swapped arrays gets its calls merged through pointer phis, which pins the
      // arrays in scratch memory). It is also the parity of u = t - t0 (every call below passes
      // P0 at even u), so each call's LDS buffers are compile-time choices.
      auto iter = [&](auto full, auto parity, int t, f32x16(&s_cur)[kKB],
                      f32x16(&s_nxt)[kKB]) __attribute__((always_inline)) {
        constexpr bool kFull = decltype(full)::value;
        constexpr int u = decltype(parity)::value;  // (t - t0) & 1
        // K(t+2) and V(t+1) go straight into the buffers this iteration does not read.
        const T* kn = kwave((u + 1) & 1);
        const T* vc = vwave(u & 1);
        if constexpr (kFull) {
          // The tiles loaded are clamped to the last one: past the end of the key range (the last
          // two steps when every tile is full) the copies land in buffers that are not read again
          // (the last step's S(t+1) is computed from a stale K buffer and discarded), which keeps
          // the tail on this branch-free body.
          const int tk = wt(min(t + 2, n_tiles - 1)), tv = wt(min(t + 1, n_tiles - 1));
          step_full(ws, s_cur, s_nxt, P, kn, vc, kl, vl, c, lane, [&] {
            dma_tile_full<false>(kbuf0 + (u & 1) * kKElems, kg, dk, tk * BC, ksn, wave);
            dma_tile_full<true>(vbuf0 + ((u + 1) & 1) * kVElems, vg, dv, tv * BC, vsn, wave);
          });
        } else {
          // LDS-DMA from inline assembly: the compiler would otherwise make the LDS reads below
          // wait for these loads, which target buffers this iteration does not read.
          if (t + 2 < n_tiles) dma_tile_asm<false>(kbuf0 + (u & 1) * kKElems, kg, dk, (t + 2) * BC, N, ksn, wave);
          if (t + 1 < n_tiles) dma_tile_asm<true>(vbuf0 + ((u + 1) & 1) * kVElems, vg, dv, (t + 1) * BC, N, vsn, wave);
          const int nv = nvalid_of(t);
          const int dg = diag_of(t, nv);
          const int nv_nxt = (t + 1 < n_tiles) ? nvalid_of(t + 1) : 0;
          if (nv_nxt > 0) qk<false>(s_nxt, ws, kn, nv_nxt, kl);
          if (nv > 0) {
            float mx = 0.f;
            const float rs = softmax_exp<false>(ws, s_cur, P, mx, nv, dg, c, lane);
            softmax_settle<false>(ws, s_cur, P, rs, mx, nv, dg, c);
            pv<false>(ws, P, vc, vl, nv, dg);
          }
        }
        wait_dma();
        __syncthreads();
      };
      using Full = std::true_type;
      using Part = std::false_type;
      using P0 = std::integral_constant<int, 0>;
      using P1 = std::integral_constant<int, 1>;
      // Tiles [0, n_full) are full for every wave and carry no diagonal (workgroup-uniform): key
      // tile t is complete below the workgroup's first row (causal) or below N. When every tile of
      // [t0, n_tiles) is full all of them take the steady step. Otherwise steady step t needs tile
      // t itself full and diagonal-free, tile t+1 inside the walk, and V(t+1) and K(t+2) whole
      // tiles inside the tensor (t + 3 <= N / BC), so that its loads need no clamp. Tile t+1 may
      // carry the causal diagonal: the steady step only computes its scores, unmasked, and the
      // partial step that exponentiates them applies the mask and the per-wave block counts.
      // Steady steps are t in [t0, n_steady).
      const int n_steady = __builtin_amdgcn_readfirstlane(walk.n_steady);
      // Unrolled by two so the S(t) / S(t+1) register sets swap roles without copies; the steady
      // loop and the tail loop get independent register assignments.
      int t = t0;
      for (; t + 1 < n_steady; t += 2) {
        iter(Full{}, P0{}, t, sa, sb);
        iter(Full{}, P1{}, t + 1, sb, sa);
      }
      if (t < n_steady) {
        iter(Full{}, P0{}, t, sa, sb);
        ++t;
        if (t < n_tiles) iter(Part{}, P1{}, t, sb, sa);
        ++t;
      }
      for (; t < n_tiles; t += 2) {
        iter(Part{}, P0{}, t, sa, sb);
        if (t + 1 < n_tiles) iter(Part{}, P1{}, t + 1, sb, sa);
      }
     }
    } else {
      f32x16 s[kKB];
      for (int t = t0; t < n_tiles; ++t) {
        dma_tile<false>(kbuf0, kg, dk, t * BC, N, ksn, wave);
        dma_tile<true>(vbuf0, vg, dv, t * BC, N, vsn, wave);
        wait_dma();
        __syncthreads();
        const int nv = nvalid_of(t);
        if (nv > 0) {
          const int dg = diag_of(t, nv);
          qk<false>(s, ws, kwave(0), nv, kl);
          float mx = 0.f;
          const float rs = softmax_exp<false>(ws, s, P, mx, nv, dg, c, lane);
          softmax_settle<false>(ws, s, P, rs, mx, nv, dg, c);
          pv<false>(ws, P, vwave(0), vl, nv, dg);
        }
        __syncthreads();
      }
    }

    // ---- merge the KS partial states of each row group (LDS is free after the last barrier) ----
    // Each wave finishes its slice of the head dim: m_fin = max_s m_s, w_s = exp2((m_s - m_fin) c),
    // O = sum_s w_s O_s and l = sum_s w_s l_s (the log-sum-exp merge of partial softmax states,
    // ref:include/fa/softmax_math.cuh:65-68; a split that saw no key of the row has m_s = -inf
    // and weighs nothing).
    auto group = [&](int gi) __attribute__((always_inline)) {
      return float4{ws.o[gi / 4][4 * (gi % 4) + 0], ws.o[gi / 4][4 * (gi % 4) + 1],
                    ws.o[gi / 4][4 * (gi % 4) + 2], ws.o[gi / 4][4 * (gi % 4) + 3]};
    };
    float4 own[kOwn];
    float m_fin, lt;
    T* stage;  // this wave's output staging: 32 rows of kStageRow elements
    if constexpr (KS > 1) {
      // Scratch: source s writes the groups of every other wave's slice, compacted (group gi at
      // gi - kOwn past its own slice), [s][rg][kGroups - kOwn][64 lanes] float4; then (m, l) per
      // [s][rg][lane].
      float4* const parts = reinterpret_cast<float4*>(lds_raw);
      float2* const mls = reinterpret_cast<float2*>(lds_raw + kPartBytes);
      auto part_at = [&](int src, int gi) {  // gi outside src's own slice
        return parts + ((src * RG + rg) * (kGroups - kOwn) + gi - (gi >= src * kOwn ? kOwn : 0)) * 64 +
               lane;
      };
#pragma unroll
      for (int gi = 0; gi < kGroups; ++gi) {
        if (gi / kOwn != ks) *part_at(ks, gi) = group(gi);
      }
      mls[(ks * RG + rg) * 64 + lane] = float2{ws.m, ws.l};
      __syncthreads();
      float ms[KS], ls[KS];
      m_fin = -__builtin_inff();
#pragma unroll
      for (int sp = 0; sp < KS; ++sp) {
        const float2 x = mls[(sp * RG + rg) * 64 + lane];
        ms[sp] = x.x;
        ls[sp] = x.y;
        m_fin = fmaxf(m_fin, x.x);
      }
      const float m_use = (m_fin == -__builtin_inff()) ? 0.f : m_fin;
      // Explicit fused multiply-adds, in split order: every tile height rounds a row the same way.
      float lsum = 0.f;
#pragma unroll
      for (int q = 0; q < kOwn; ++q) own[q] = float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sp = 0; sp < KS; ++sp) {
        const float w = exp2_hw((ms[sp] - m_use) * c);
        lsum = __builtin_fmaf(ls[sp], w, lsum);
#pragma unroll
        for (int q = 0; q < kOwn; ++q) {
          float4 x;
          if (sp == ks) {
            x = group(q);
#pragma unroll
            for (int kk = 1; kk < KS; ++kk) {
              if (ks == kk) x = group(kk * kOwn + q);
            }
          } else {
            x = *part_at(sp, ks * kOwn + q);
          }
          own[q] = float4{__builtin_fmaf(x.x, w, own[q].x), __builtin_fmaf(x.y, w, own[q].y),
                          __builtin_fmaf(x.z, w, own[q].z), __builtin_fmaf(x.w, w, own[q].w)};
        }
      }
      lt = halves_sum(lsum);
      // Staging: this wave's slice in the scratch of source 0 (1 if this is wave 0), which no other
      // wave reads; the reads above were issued first, and one wave's LDS operations complete in
      // order.
      stage = reinterpret_cast<T*>(part_at(ks == 0 ? 1 : 0, ks * kOwn) - lane);
    } else {
#pragma unroll
      for (int q = 0; q < kOwn; ++q) own[q] = group(q);
      m_fin = ws.m;
      lt = halves_sum(ws.l);
      stage = reinterpret_cast<T*>(lds_raw) + static_cast<size_t>(wave) * 32 * kStageRow;
    }

    // ---- epilogue: O = acc / l, lse = m*scale + ln l (ref:include/fa/softmax_math.cuh:58-71) ----
    if (!wave_valid) return;
    const float inv = (lt > 0.f) ? 1.f / lt : 0.f;
    const int d0 = ks * kSliceD;  // first head-dim entry of this wave's slice
    if (S > 1) {
      // One part of a split walk: its normalised O in fp32 and its LSE (-inf when the part saw
      // no key) for fa_s5_combine.
      const size_t prow =
          ((static_cast<size_t>(part) * a.B + b) * a.H + h) * static_cast<size_t>(N) + row;
      float* op = a.o_part + prow * D + d0;
#pragma unroll
      for (int q = 0; q < kOwn; ++q) {
        *reinterpret_cast<float4*>(op + 8 * q + 4 * g) = own[q] * inv;
      }
      if (ks == 0 && g == 0) {
        a.lse_part[prow] = (lt > 0.f && m_fin != -__builtin_inff())
                               ? m_fin * a.scale + log2_hw(lt) * kLn2
                               : -__builtin_inff();
      }
      return;
    }
    // Through LDS to whole-row stores: lane (row, g) writes its 4 entries of each group, then every
    // lane stores 16 contiguous bytes, consecutive lanes along a row's slice. The stores are
    // non-temporal: nothing in this launch reads O, and rows written whole need no merging in L2
    // (measured against plain stores on cache-cold inputs: C128 -1.9 %, C128 causal -2.9 %, LONG
    // at N 512 -4.5 %, C64 and LONG unchanged).
#pragma unroll
    for (int q = 0; q < kOwn; ++q) {
      const float4 x = own[q] * inv;
      T* dst = stage + (lane & 31) * kStageRow + 8 * q + 4 * g;
      if constexpr (kF16) {
        *reinterpret_cast<f16x4*>(dst) =
            f16x4{(_Float16)x.x, (_Float16)x.y, (_Float16)x.z, (_Float16)x.w};
      } else {
        *reinterpret_cast<bf16x4*>(dst) = bf16x4{(__bf16)x.x, (__bf16)x.y, (__bf16)x.z, (__bf16)x.w};
      }
    }
    T* const obase = static_cast<T*>(a.o) + b * a.osb + h * a.osh + r0 * a.osn + d0;
#pragma unroll
    for (int i = 0; i < kOwn / 2; ++i) {
      const int ch = i * 64 + lane;
      const int r = ch / kOwn, cc = ch % kOwn;
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(stage + r * kStageRow + 8 * cc),
                                  reinterpret_cast<u32x4*>(obase + r * a.osn + 8 * cc));
    }
    if (ks == 0 && g == 0) {
      a.lse[(static_cast<size_t>(b) * a.H + h) * static_cast<size_t>(N) + row] =
          (lt > 0.f && m_fin != -__builtin_inff()) ? m_fin * a.scale + log2_hw(lt) * kLn2
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

// Merge of the parts of split key walks: per row, L* = max_s LSE_s, w_s = exp(LSE_s - L*),
// O = sum_s w_s O_s / sum_s w_s and LSE = L* + ln sum_s w_s (the log-sum-exp merge of partial
// softmax states, ref:include/fa/softmax_math.cuh:65-68; empty parts carry LSE_s = -inf and weigh
// nothing). One thread per four head-dim elements of a row; fp32 throughout, one rounding to T.
// Every part's LSE and partial O are loaded before the first is used (the part loop is unrolled
// to kMaxSplitParts and predicated on n_splits), so the kernel waits for memory once, not once
// per part and pass.
template <typename T, int D>
__global__ __launch_bounds__(256) void fa_s5_combine(KArgs a) {
  constexpr int kTpr = D / 4;  // threads per row
  constexpr int kRows = 256 / kTpr;
  constexpr float kLog2e = 1.44269504088896341f;
  const long long rows = static_cast<long long>(a.B) * a.H * a.N;
  const long long r = static_cast<long long>(blockIdx.x) * kRows + threadIdx.x / kTpr;
  if (r >= rows) return;
  const int d = 4 * (threadIdx.x % kTpr);
  const int S = a.n_splits;
  float ls[kMaxSplitParts];
  float4 po[kMaxSplitParts];
#pragma unroll
  for (int sp = 0; sp < kMaxSplitParts; ++sp) {
    if (sp < S) {
      ls[sp] = a.lse_part[sp * rows + r];
      po[sp] = *reinterpret_cast<const float4*>(a.o_part + (sp * rows + r) * D + d);
    }
  }
  float lmax = -__builtin_inff();
#pragma unroll
  for (int sp = 0; sp < kMaxSplitParts; ++sp) {
    if (sp < S) lmax = fmaxf(lmax, ls[sp]);
  }
  const long long bh = r / a.N;
  const int n = static_cast<int>(r - bh * a.N);
  const int b = static_cast<int>(bh / a.H);
  const int h = static_cast<int>(bh - static_cast<long long>(b) * a.H);
  T* orow = static_cast<T*>(a.o) + b * a.osb + h * a.osh + static_cast<long long>(n) * a.osn + d;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float sum = 0.f;
  if (lmax != -__builtin_inff()) {
#pragma unroll
    for (int sp = 0; sp < kMaxSplitParts; ++sp) {
      if (sp < S) {
        const float w = exp2_hw((ls[sp] - lmax) * kLog2e);
        sum += w;
        acc[0] = __builtin_fmaf(w, po[sp].x, acc[0]);
        acc[1] = __builtin_fmaf(w, po[sp].y, acc[1]);
        acc[2] = __builtin_fmaf(w, po[sp].z, acc[2]);
        acc[3] = __builtin_fmaf(w, po[sp].w, acc[3]);
      }
    }
  }
  // A row no part saw (impossible for a non-empty walk) keeps O = 0 and LSE = +inf.
  const float inv = sum > 0.f ? 1.f / sum : 0.f;
  if constexpr (__is_same(T, _Float16)) {
    *reinterpret_cast<f16x4*>(orow) = f16x4{(_Float16)(acc[0] * inv), (_Float16)(acc[1] * inv),
                                            (_Float16)(acc[2] * inv), (_Float16)(acc[3] * inv)};
  } else {
    *reinterpret_cast<bf16x4*>(orow) = bf16x4{(__bf16)(acc[0] * inv), (__bf16)(acc[1] * inv),
                                              (__bf16)(acc[2] * inv), (__bf16)(acc[3] * inv)};
  }
  if (d == 0) a.lse[r] = sum > 0.f ? lmax + log2_hw(sum) * kLn2 : __builtin_inff();
}

template <typename T, int D>
int launch_combine(const KArgs& a, hipStream_t stream) {
  constexpr int kRows = 256 / (D / 4);
  const long long rows = static_cast<long long>(a.B) * a.H * a.N;
  const long long grid = (rows + kRows - 1) / kRows;
  if (a.n_splits < 2 || a.n_splits > kMaxSplitParts || a.o_part == nullptr ||
      a.lse_part == nullptr || grid <= 0 || grid > 0x7fffffffLL) {
    return static_cast<int>(hipErrorInvalidValue);
  }
  hipLaunchKernelGGL((fa_s5_combine<T, D>), dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                     stream, a);
  return static_cast<int>(hipGetLastError());
}

// Workgroups of one variant resident per CU at once (the runtime's occupancy for its registers and
// LDS), asked once per process; 1 if the query fails.
template <int STAGE, typename T, int D, int RG, int KS, int BCW>
int resident_per_cu() {
  static const int n = [] {
    int blocks = 0;
    hipError_t e;
    if constexpr (STAGE == 5) {
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fa_s5_tuned<T, D, RG, KS, BCW>,
                                                       64 * RG * KS, 0);
    } else {
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fa_s4_mfma<T, D, RG, KS, BCW>,
                                                       64 * RG * KS, 0);
    }
    return (e == hipSuccess && blocks > 0) ? blocks : 1;
  }();
  return n;
}

// Host-side launch of one instantiated variant (STAGE 5 or 4).
template <int STAGE, typename T, int D, int RG, int KS, int BCW>
int launch(const KArgs& in, hipStream_t stream) {
  using A = Fa16<T, D, RG, KS, BCW, STAGE == 5>;
  KArgs a = in;
  a.n_qtiles = (a.N + A::kBr - 1) / A::kBr;
  a.fd_qtiles = make_fastdiv(static_cast<uint32_t>(a.n_qtiles));
  a.xcd_heads = layout::xcd_heads_for(a.B * a.H, a.causal != 0);
  a.fd_xcd_heads = make_fastdiv(static_cast<uint32_t>(a.xcd_heads > 0 ? a.xcd_heads : 1));
  const long long grid = static_cast<long long>(a.n_qtiles) * a.B * a.H * a.n_splits;
  // The snake order pays only when the whole grid is resident at once (every CU's workgroups are
  // the ones the dispatcher handed out in its first rounds); once workgroups wait for free slots,
  // the dispatcher itself balances the plain longest-first order better.
  if (a.xcd_heads == 0 || a.n_splits != 1 ||
      grid > static_cast<long long>(resident_per_cu<STAGE, T, D, RG, KS, BCW>()) * a.xcd_cus *
                 layout::kXcds) {
    a.xcd_cus = 0;
  }
  a.fd_xcd_cus = make_fastdiv(static_cast<uint32_t>(a.xcd_cus > 0 ? a.xcd_cus : 1));
  if (a.n_splits < 1 || (a.n_splits > 1 && (STAGE != 5 || a.o_part == nullptr ||
                                            a.lse_part == nullptr))) {
    return static_cast<int>(hipErrorInvalidValue);
  }
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
  return Variant{D, 32 * RG, KS * BCW, &launch<STAGE, T, D, RG, KS, BCW>, RG * KS};
}

// ---- instantiation tables: one (RG, KS, BCW) per (BR, BC) -------------------------------------
// Stage 5 rows cover the default tiles, the sweep set and the tile-invariance set, including
// key-split variants at every height so the merge path is tested at small N. Every row fits the
// register budget of its occupancy without spills or scratch (256 VGPRs per wave at 8 waves per
// workgroup; tests/test_register_budget_cpu.py checks the compiler's report for every kernel);
// that is what rules out BCW = 64 at D = 128 with 8 waves, BR 256 / BC 128, and BR 256 / BC 64 at
// D = 128 (8 x 32 rows with 64 keys per wave: 53 registers spilled to scratch).
template <typename T, int D, int STAGE>
struct S5Rows {
  static constexpr Variant rows[] = {
      variant<STAGE, T, D, 1, 1, 32>(),  // BR  32, BC  32
      variant<STAGE, T, D, 1, 2, 32>(),  // BR  32, BC  64 (2-way split)
      variant<STAGE, T, D, 2, 1, 32>(),  // BR  64, BC  32
      variant<STAGE, T, D, 2, 2, 32>(),  // BR  64, BC  64 (2-way split)
      variant<STAGE, T, D, 4, 1, 32>(),  // BR 128, BC  32
      variant<STAGE, T, D, 4, 2, 32>(),  // BR 128, BC  64 (2-way split) -- D = 128 default
  };
};

// Per head dim, the tiles with 64 keys per wave or four key splits:
//   D = 64:  BR 64 / 128 / 32 x BC 128 (2 key splits of 64 keys; BR 128 is the D = 64 default),
//            BR 256 / BC 64, and BR 32 / 64 x BC 256 (4 key splits of 64 keys);
//   D = 128: BR 32 / 64 x BC 128 (4 key splits of 32 keys).
// The four-split tiles serve grids of at most one workgroup per CU, where two splits would leave
// SIMDs with one wave or none.
// STAGE 5 is the table stage 5 launches; STAGE 4 gives the same tiles with the synchronous loop
// (launched as fa_s4_mfma), which stage 5 runs under FA_S5_PREFETCH=0.
template <typename T, int STAGE = 5>
VariantList s5_table() {
  using R64 = S5Rows<T, 64, STAGE>;
  using R128 = S5Rows<T, 128, STAGE>;
  static const Variant t[] = {
      R64::rows[0],  R64::rows[1],  R64::rows[2],  R64::rows[3],
      R64::rows[4],  R64::rows[5],  variant<STAGE, T, 64, 2, 2, 64>(),
      variant<STAGE, T, 64, 8, 1, 64>(),  variant<STAGE, T, 64, 4, 2, 64>(),
      variant<STAGE, T, 64, 1, 2, 64>(),  variant<STAGE, T, 64, 1, 4, 64>(),
      variant<STAGE, T, 64, 2, 4, 64>(),
      R128::rows[0], R128::rows[1], R128::rows[2], R128::rows[3],
      R128::rows[4], R128::rows[5], variant<STAGE, T, 128, 1, 4, 32>(),
      variant<STAGE, T, 128, 2, 4, 32>()};
  return VariantList{t, static_cast<int>(sizeof(t) / sizeof(t[0]))};
}

// Stage 4: BR fixed at 128 (4 row groups), BC in {32, 64, 128}.
template <typename T>
VariantList s4_table() {
  static const Variant t[] = {variant<4, T, 64, 4, 1, 32>(),  variant<4, T, 64, 4, 2, 32>(),
                              variant<4, T, 64, 4, 2, 64>(),  variant<4, T, 128, 4, 1, 32>(),
                              variant<4, T, 128, 4, 2, 32>(), variant<4, T, 128, 4, 2, 64>()};
  return VariantList{t, static_cast<int>(sizeof(t) / sizeof(t[0]))};
}

}  // namespace m16
}  // namespace fa
