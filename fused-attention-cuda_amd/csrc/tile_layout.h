// tile_layout.h -- the integer layout of the stage-4/5 kernels' K/V tiles: which global element
// every lane of every LDS-DMA instruction copies, where a tile lives in LDS, which LDS bytes each
// MFMA operand read touches, and which key tiles a workgroup walks and loads.
//
// Pure integer functions with no HIP intrinsics, compiled for the device by attn_mfma16.h and for
// the host by tests/address_model.cpp, which replays every load of every workgroup on the CPU and
// checks that each global read stays inside its tensor and each LDS access inside its buffer (the
// role of the reference's compute-sanitizer memcheck run, ref:scripts/gpu_run.sh:157-181).
#pragma once

#if defined(__HIPCC__) || defined(__HIP__)
#define FA_HD __host__ __device__
#else
#define FA_HD
#endif

namespace fa {
namespace layout {

// LDS layout of a K/V tile: BC rows of D 16-bit elements, unpadded; the 16-byte chunk c of row r
// lives at chunk position c ^ swz(r). The swizzles were chosen by the measured read rate of each
// operand pattern on gfx950: K rows are read 16 consecutive rows per 16 lanes (ds_read_b128), so
// D = 64 rows (128 bytes) pair up, (r >> 1) & 7, and D = 128 rows use r & 15; V is read through
// the transpose path 4 consecutive rows per 16 lanes, 2 (r & 3) at D = 64 and 4 (r & 3) at
// D = 128. Every swizzle depends on r % 32 only, so a lane's offsets inside a 32-key block are
// loop-invariant.
template <int D, bool IS_V>
FA_HD constexpr int swz(int row) {
  if constexpr (IS_V) {
    return (D == 64 ? 2 : 4) * (row & 3);
  } else {
    return D == 64 ? ((row >> 1) & 7) : (row & 15);
  }
}

// LDS-DMA: instruction j of a tile covers chunk positions [64 j, 64 j + 64) (1 KiB) and goes to
// wave j % waves; lane l writes position 64 j + l, so it copies the global chunk whose swizzled
// position that is. Its source relative to the tile's first key: tile-local row `row` and element
// offset `off` = row * sn + 8 * (its chunk in the row) for a row stride of sn elements.
template <int D, bool IS_V>
struct DmaSrc {
  int row;
  int off;
};
template <int D, bool IS_V>
FA_HD inline DmaSrc<D, IS_V> dma_src(int waves, int wave, int lane, int i, int sn) {
  constexpr int kRowChunks = D / 8;
  const int pos = 64 * (wave + i * waves) + lane;  // chunk position in the tile
  const int row = pos / kRowChunks;
  return DmaSrc<D, IS_V>{row, row * sn + 8 * ((pos % kRowChunks) ^ swz<D, IS_V>(row))};
}

// K operand of S^T = K Q^T, head-dim step st: lane l reads key row l % 32 of a 32-key block,
// chunk 2 st + l / 32 (head-dim 16 st + 8 (l / 32)); element offset inside the block.
template <int D>
FA_HD constexpr int k_operand_offset(int lane, int st) {
  return (lane & 31) * D + 8 * ((2 * st + (lane >> 5)) ^ swz<D, false>(lane & 31));
}

// V^T operand through the transpose read, head-dim block db: lane l = 16 G + 4 j + q addresses key
// row 4 (G / 2) + j of a 16-key group (and 8 rows further for the second read) at head-dim
// 32 db + 16 (G % 2) + 4 q; element offset inside the group.
template <int D>
FA_HD constexpr int v_operand_offset(int lane, int db) {
  const int G = lane >> 4, j = (lane >> 2) & 3, q = lane & 3;
  const int chunk = (4 * db + 2 * (G & 1) + (q >> 1)) ^ swz<D, true>(j);
  return (4 * (G >> 1) + j) * D + 8 * chunk + 4 * (q & 1);
}

// The key tiles one stage-5 workgroup walks: [t0, n_tiles) of BC keys (its part of the query
// tile's walk when the walk is split into `splits` parts), and n_steady: steps t in
// [t0, n_steady) take the branch-free steady body, whose loads (K(t+2), V(t+1), clamped to the last
// tile of the walk) are whole tiles inside the tensor. The rule, in the kernel's words: when every
// tile of the walk is full, all of them take the steady step; otherwise step t needs tile t full
// and free of the causal diagonal, t + 1 inside the walk, and t + 3 <= N / BC.
//
// Walk order. Tiles are walked in the order walk_tile(w, t0), walk_tile(w, t0 + 1), ...: the
// range [t0, rot_end) rotated left by `rot` (0 <= rot < rot_end - t0; rot_end <= n_steady), then
// the rest in order. Workgroups that share a head's K/V start their rotations at different tiles,
// so that a tile one of them fetches from HBM is found in L2 by the others a few steps later
// instead of all of them waiting on the same miss at once (rotate_walk).
struct Walk {
  int t0;
  int n_tiles;
  int n_steady;
  int rot;
  int rot_end;
};
FA_HD inline int walk_tile(const Walk& w, int t) {
  if (t >= w.rot_end) return t;
  const int x = t + w.rot;
  return x < w.rot_end ? x : x - (w.rot_end - w.t0);
}
// div_splits(x) must return x / splits (the kernel passes its multiply-shift division).
template <typename DivSplits>
FA_HD inline Walk plan_walk(int N, int BC, int BR, int qt, bool causal, int part,
                            DivSplits div_splits) {
  const int i0 = qt * BR;
  const int kv_end = causal ? (N < i0 + BR ? N : i0 + BR) : N;
  const int n_walk = (kv_end + BC - 1) / BC;
  Walk w;
  w.rot = 0;
  w.rot_end = 0;
  w.t0 = div_splits(part * n_walk);
  w.n_tiles = div_splits((part + 1) * n_walk);
  const int n_full = (causal ? i0 : N) / BC;
  if (n_full >= w.n_tiles) {
    w.n_steady = w.n_tiles;
  } else {
    int s = w.n_tiles - 1 < n_full ? w.n_tiles - 1 : n_full;
    s = s < N / BC - 2 ? s : N / BC - 2;
    w.n_steady = s > w.t0 ? s : w.t0;
  }
  return w;
}

// The rotation of a workgroup's walk. It is a property of the 128-row block (kRotRows) that holds
// the workgroup's first row, so that every workgroup height (32, 64 or 128 rows) gives each 32-row
// wave the same sequence of key tiles, hence the same results: the rotated range is the block's
// steady range [t0, n_steady of a 128-row workgroup at the block), which lies inside the steady
// range of any shorter workgroup of the block. With groups_lg < 0 block blk of n_blocks starts
// blk / n_blocks of the way round it; with groups_lg = k the blocks form 2^k groups of consecutive
// blocks, and group g = floor(blk 2^k / n_blocks) starts g / 2^k of the way round. div_blocks(x)
// must return x / n_blocks, n_blocks = ceil(N / kRotRows).
constexpr int kRotRows = 128;
template <typename DivSplits, typename DivBlocks>
FA_HD inline void rotate_walk(Walk& w, int N, int BC, int BR, int qt, bool causal, int part,
                              DivSplits div_splits, DivBlocks div_blocks, int groups_lg = -1) {
  const int blk = qt * BR / kRotRows;
  const Walk wb = plan_walk(N, BC, kRotRows, blk, causal, part, div_splits);
  const int end = wb.n_steady < w.n_steady ? wb.n_steady : w.n_steady;
  if (wb.t0 != w.t0 || end - w.t0 < 2) return;
  w.rot_end = end;
  if (groups_lg < 0) {
    w.rot = div_blocks(blk * (end - w.t0));
  } else {
    const int g = div_blocks(blk << groups_lg);  // the block's group, 0 .. 2^groups_lg - 1
    w.rot = (g * (end - w.t0)) >> groups_lg;
  }
}

// The work item of workgroup `bid` of a stage-4/5 grid of G = n_qtiles * BH * splits workgroups
// (BH = B * H): its batch-head bh, query tile qt and part of a split walk. The hardware hands
// workgroup i to XCD (i + c) % kXcds, with c the same for every workgroup of a launch (the
// dispatcher's round robin goes on from where earlier launches left it; XCC_ID read on the box
// showed c = 0, 5, 6 and 7), so workgroups with equal i % kXcds share an XCD, and each XCD has its
// own L2. Each XCD therefore receives a contiguous range of items and fetches a head's K/V into
// one L2. Inside an XCD's range:
//  - head-major (xcd_heads == 0): items (bh, qt, part) in order;
//  - tile-major (xcd_heads = BH / kXcds, only when kXcds divides BH): the range is xcd_heads
//    whole heads, issued one query tile of all of them at a time. On a causal grid that issues
//    the range's longest walks first (list scheduling, longest first); head-major issues them
//    head by head, so the long tiles of an XCD's last heads start after the short tiles of its
//    first ones.
// Causal grids count qt down, longest key walk first. The parts of one query tile are
// consecutive items in both orders. div_*(x) must return x / splits, x / n_qtiles and
// x / xcd_heads (the kernel passes its multiply-shift divisions).
constexpr int kXcds = 8;
struct Item {
  int bh;
  int qt;
  int part;
};
//
// Snake order (xcd_cus > 0, tile-major and unsplit only): the dispatcher fills an XCD's CUs one
// workgroup each, in order, before it gives any CU a second one, so with several resident
// workgroups per CU the i-th workgroup of every round of xcd_cus shares a CU. Every second round
// is issued in reverse, so that the longest query tile of the first round shares its CU with the
// shortest of the second (32 + 1, 31 + 2, ... key tiles instead of 32 + 16, 31 + 15, ...).
// div_cus(x) must return x / xcd_cus.
template <typename DivS, typename DivQ, typename DivX, typename DivC>
FA_HD inline Item grid_item(int bid, int G, int n_qtiles, int splits, bool causal, int xcd_heads,
                            int xcd_cus, DivS div_splits, DivQ div_qtiles, DivX div_xcd_heads,
                            DivC div_cus) {
  const int xcd = bid % kXcds;
  int local = bid / kXcds;
  Item it;
  int q;
  if (xcd_heads > 0) {
    if (xcd_cus > 0 && splits == 1) {
      const int round = div_cus(local);
      const int first = round * xcd_cus;
      const int per_xcd = G / kXcds;
      const int len = per_xcd - first < xcd_cus ? per_xcd - first : xcd_cus;
      if (round & 1) local = first + (len - 1 - (local - first));
    }
    const int item = div_splits(local);
    it.part = local - item * splits;
    q = div_xcd_heads(item);
    it.bh = xcd * xcd_heads + (item - q * xcd_heads);
  } else {
    const int per = G / kXcds, rem = G % kXcds;
    const int logical = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + local;
    const int item = div_splits(logical);
    it.part = logical - item * splits;
    it.bh = div_qtiles(item);
    q = item - it.bh * n_qtiles;
  }
  it.qt = causal ? n_qtiles - 1 - q : q;
  return it;
}

// The launcher's choice of order: tile-major on causal grids whose BH splits into whole heads per
// XCD, two or more of them (with one the orders coincide); head-major otherwise, where every
// walk has the same length and the order only decides which heads share an L2.
FA_HD constexpr int xcd_heads_for(int BH, bool causal) {
  return (causal && BH % kXcds == 0 && BH / kXcds > 1) ? BH / kXcds : 0;
}

}  // namespace layout
}  // namespace fa
