// CPU replay of every global read and LDS access of the stage-4/5 and decode kernels' K/V paths,
// built from the kernels' own layout functions (csrc/tile_layout.h) and run by
// tests/test_address_model_cpu.py. For each tile variant (D, RG, KS, BCW) given on the command
// line and each problem of a sweep -- N (full and partial tiles), causal or not, split walks of
// 1..16 parts, dense and strided rows -- it walks every workgroup through the kernel's load
// schedule (prologue, steady steps with their clamped tile indices, partial steps) and checks:
//   * every LDS-DMA source element range lies inside its [N, D] head of K or V: rows past the end
//     of the keys are clamped to row N - 1, and the steady step's unclamped loads are whole tiles
//     inside the tensor;
//   * every LDS-DMA destination lies inside its tile buffer, and one tile's DMA writes each
//     16-byte chunk of the buffer exactly once (no valid row is left unwritten);
//   * every MFMA operand read (K rows, V^T transpose reads) lies inside the tile buffer;
//   * stage 5's Q tile (BR rows in the K layout, rows past N clamped to N - 1) is read from inside
//     its [N, D] head and written once per chunk into its LDS region, and each wave's Q register
//     reads from that region stay inside it;
//   * a split part's partial rows lie inside the workspace the library sizes for it.
// Decode's split kernel (attn_decode.h) is replayed the same way: each split's keys [k_begin,
// k_end) in 128-key tiles with the last tile clamped to the split's last key. The grid decode
// (layout::grid_item) is checked to hand every workgroup a distinct in-range work item.
// Exits non-zero on the first violation, printing the case.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "tile_layout.h"

namespace {

struct Variant {
  int D, RG, KS, BCW;
};

long long g_checks = 0;
bool g_plant_no_clamp = false;  // test of the checker itself: drop the row clamp of every load

[[noreturn]] void fail(const std::string& what) {
  std::printf("VIOLATION: %s\n", what.c_str());
  std::exit(1);
}

std::string ctx(const Variant& v, int N, int sn, bool causal, int S, int part, int qt) {
  char buf[256];
  std::snprintf(buf, sizeof(buf), "D=%d RG=%d KS=%d BCW=%d N=%d sn=%d causal=%d S=%d part=%d qt=%d",
                v.D, v.RG, v.KS, v.BCW, N, sn, causal ? 1 : 0, S, part, qt);
  return buf;
}

// One tile load of one tensor: every wave's DMA instructions, every lane.
template <int D, bool IS_V>
void check_tile_load(const Variant& v, int N, int sn, int k0, bool clamp, const std::string& c) {
  const int waves = v.RG * v.KS;
  const int BC = v.KS * v.BCW;
  const int chunks = BC * D / 8;
  const int per_wave = chunks / 64 / waves;
  const long long head_end = static_cast<long long>(N - 1) * sn + D;  // one past the last element
  if (g_plant_no_clamp) clamp = false;
  if (!clamp && k0 + BC > N && !g_plant_no_clamp) fail("unclamped load of a partial tile: " + c);
  std::vector<int> written(chunks, 0);
  for (int w = 0; w < waves; ++w) {
    for (int i = 0; i < per_wave; ++i) {
      for (int lane = 0; lane < 64; ++lane) {
        const auto src = fa::layout::dma_src<D, IS_V>(waves, w, lane, i, sn);
        long long off = src.off;
        if (clamp) {
          const int last = src.row < N - 1 - k0 ? src.row : N - 1 - k0;
          off += static_cast<long long>(last - src.row) * sn;
        }
        const long long elem = static_cast<long long>(k0) * sn + off;
        if (elem < 0 || elem + 8 > head_end) {
          fail("DMA source outside the head (" + std::to_string(elem) + ".." +
               std::to_string(elem + 8) + " of " + std::to_string(head_end) + "): " + c);
        }
        const int pos = 64 * (w + i * waves) + lane;
        if (pos < 0 || pos >= chunks) fail("DMA destination outside the tile buffer: " + c);
        ++written[pos];
        ++g_checks;
      }
    }
  }
  for (int p = 0; p < chunks; ++p) {
    if (written[p] != 1) fail("tile chunk " + std::to_string(p) + " written " +
                              std::to_string(written[p]) + " times: " + c);
  }
}

// MFMA operand reads of one wave of key split ks inside one tile buffer (element offsets).
template <int D>
void check_operand_reads(const Variant& v) {
  const int BC = v.KS * v.BCW;
  const int elems = BC * D;
  for (int ks = 0; ks < v.KS; ++ks) {
    const int kbase = ks * v.BCW * D;
    for (int kb = 0; kb < v.BCW / 32; ++kb) {
      for (int lane = 0; lane < 64; ++lane) {
        for (int st = 0; st < D / 16; ++st) {
          const int e = kbase + 32 * kb * D + fa::layout::k_operand_offset<D>(lane, st);
          if (e < 0 || e + 8 > elems) fail("K operand read outside the tile buffer");
          ++g_checks;
        }
        for (int h = 0; h < 2; ++h) {
          for (int db = 0; db < D / 32; ++db) {
            const int base = kbase + (32 * kb + 16 * h) * D + fa::layout::v_operand_offset<D>(lane, db);
            for (int second = 0; second < 2; ++second) {
              const int e = base + second * 8 * D;
              if (e < 0 || e + 4 > elems) fail("V^T operand read outside the tile buffer");
              ++g_checks;
            }
          }
        }
      }
    }
  }
}

// Stage 5's Q tile: rows [qt * BR, qt * BR + BR) of the head (row stride sn), K layout, through
// every wave's LDS-DMA; then each wave's Q operand reads (its 32-row block).
template <int D>
void check_q_load(const Variant& v, int N, int sn, int qt, const std::string& c) {
  const int waves = v.RG * v.KS;
  const int BR = 32 * v.RG;
  const int chunks = BR * D / 8;
  if (chunks % (64 * waves) != 0) fail("Q tile is not whole DMA instructions per wave: " + c);
  const int per_wave = chunks / 64 / waves;
  const long long head_end = static_cast<long long>(N - 1) * sn + D;
  const int i0 = qt * BR;
  std::vector<int> written(chunks, 0);
  for (int w = 0; w < waves; ++w) {
    for (int i = 0; i < per_wave; ++i) {
      for (int lane = 0; lane < 64; ++lane) {
        const auto src = fa::layout::dma_src<D, false>(waves, w, lane, i, sn);
        int qrow = i0 + src.row;
        if (!g_plant_no_clamp && qrow > N - 1) qrow = N - 1;
        const long long elem = static_cast<long long>(i0) * sn + src.off +
                               static_cast<long long>(qrow - i0 - src.row) * sn;
        if (elem < 0 || elem + 8 > head_end) fail("Q DMA source outside the head: " + c);
        const int pos = 64 * (w + i * waves) + lane;
        if (pos < 0 || pos >= chunks) fail("Q DMA destination outside the Q region: " + c);
        ++written[pos];
        ++g_checks;
      }
    }
  }
  for (int p = 0; p < chunks; ++p) {
    if (written[p] != 1) fail("Q chunk " + std::to_string(p) + " written " +
                              std::to_string(written[p]) + " times: " + c);
  }
  for (int rg = 0; rg < v.RG; ++rg) {
    for (int lane = 0; lane < 64; ++lane) {
      for (int st = 0; st < D / 16; ++st) {
        const int e = 32 * rg * D + fa::layout::k_operand_offset<D>(lane, st);
        if (e < 0 || e + 8 > BR * D) fail("Q operand read outside the Q region: " + c);
        ++g_checks;
      }
    }
  }
}

// The load schedule of one stage-5 (pipelined) or stage-4 (synchronous) workgroup.
template <int D>
void replay_workgroup(const Variant& v, int N, int sn, bool causal, int S, int part, int qt,
                      bool pipelined, bool rotate, int groups_lg = -1) {
  const int BC = v.KS * v.BCW, BR = 32 * v.RG;
  auto walk = fa::layout::plan_walk(N, BC, BR, qt, causal, part, [S](int x) { return x / S; });
  const int n_blocks = (N + fa::layout::kRotRows - 1) / fa::layout::kRotRows;
  if (rotate && pipelined) {
    fa::layout::rotate_walk(walk, N, BC, BR, qt, causal, part, [S](int x) { return x / S; },
                            [n_blocks](int x) { return x / n_blocks; }, groups_lg);
  }
  auto wt = [&](int t) { return fa::layout::walk_tile(walk, t); };
  const std::string c = ctx(v, N, sn, causal, S, part, qt);
  if (walk.t0 > walk.n_tiles || walk.n_steady < walk.t0 || walk.n_steady > walk.n_tiles ||
      walk.rot < 0 || walk.rot_end > walk.n_steady ||
      (walk.rot > 0 && walk.rot >= walk.rot_end - walk.t0)) {
    fail("inconsistent walk plan: " + c);
  }
  // The rotated order visits every tile of the walk exactly once.
  {
    std::vector<int> seen(walk.n_tiles, 0);
    for (int t = walk.t0; t < walk.n_tiles; ++t) {
      const int k = wt(t);
      if (k < walk.t0 || k >= walk.n_tiles || seen[k]++) fail("walk order is not a permutation: " + c);
      if ((t < walk.n_steady) != (k < walk.n_steady)) fail("rotation leaves the steady range: " + c);
      ++g_checks;
    }
  }
  if (walk.t0 == walk.n_tiles) return;  // an empty part of a split walk loads nothing
  if (!pipelined) {
    for (int t = walk.t0; t < walk.n_tiles; ++t) {
      check_tile_load<D, false>(v, N, sn, t * BC, true, c);
      check_tile_load<D, true>(v, N, sn, t * BC, true, c);
    }
    return;
  }
  // Prologue: Q, K(t0), V(t0), K(t0 + 1).
  check_q_load<D>(v, N, sn, qt, c + " (Q)");
  check_tile_load<D, false>(v, N, sn, wt(walk.t0) * BC, true, c);
  check_tile_load<D, true>(v, N, sn, wt(walk.t0) * BC, true, c);
  if (walk.t0 + 1 < walk.n_tiles) check_tile_load<D, false>(v, N, sn, wt(walk.t0 + 1) * BC, true, c);
  for (int t = walk.t0; t < walk.n_tiles; ++t) {
    if (t < walk.n_steady) {
      // Steady step: K(t + 2) and V(t + 1) clamped to the walk's last tile, loaded unclamped.
      const int tk = wt(t + 2 < walk.n_tiles - 1 ? t + 2 : walk.n_tiles - 1);
      const int tv = wt(t + 1 < walk.n_tiles - 1 ? t + 1 : walk.n_tiles - 1);
      check_tile_load<D, false>(v, N, sn, tk * BC, false, c + " (steady K)");
      check_tile_load<D, true>(v, N, sn, tv * BC, false, c + " (steady V)");
    } else {
      if (t + 2 < walk.n_tiles) check_tile_load<D, false>(v, N, sn, (t + 2) * BC, true, c);
      if (t + 1 < walk.n_tiles) check_tile_load<D, true>(v, N, sn, (t + 1) * BC, true, c);
    }
  }
}

// Split walks: part p's partial rows [S, B, H, N, D] (one head here) inside the workspace.
void check_split_rows(int N, int D, int S, int part, int rows_lo, int rows_hi) {
  const long long total = static_cast<long long>(S) * N * D;
  const long long lo = (static_cast<long long>(part) * N + rows_lo) * D;
  const long long hi = (static_cast<long long>(part) * N + rows_hi) * D;  // exclusive
  if (lo < 0 || hi > total) fail("split partial rows outside the workspace");
  ++g_checks;
}

template <int D>
void sweep_variant(const Variant& v) {
  check_operand_reads<D>(v);
  const int BC = v.KS * v.BCW, BR = 32 * v.RG;
  std::vector<int> lengths = {32, 64, 96, 160, 288, 320};
  for (int m : {1, 3, 5, 7, 9}) lengths.push_back(m * BC);
  for (int m : {1, 3, 5}) lengths.push_back(m * BC + 32);
  for (int m : {2, 4}) lengths.push_back(m * BC - 32);
  for (int N : lengths) {
    if (N < 32 || N % 32 != 0) continue;
    for (int sn : {D, 3 * 4 * D + 8}) {  // dense rows, and rows of a strided [B, N, 3, H, D] view
      for (bool causal : {false, true}) {
        const int n_qtiles = (N + BR - 1) / BR;
        for (int S : {1, 2, 3, 5, 16}) {
          for (int part = 0; part < S; ++part) {
            for (int qt = 0; qt < n_qtiles; ++qt) {
              replay_workgroup<D>(v, N, sn, causal, S, part, qt, true, false);
              for (const int groups_lg : {-1, 1, 2}) {  // one start per block, 2 or 4 groups
                replay_workgroup<D>(v, N, sn, causal, S, part, qt, true, true, groups_lg);
              }
              if (S == 1) replay_workgroup<D>(v, N, sn, causal, 1, 0, qt, false, false);
              if (S > 1) check_split_rows(N, D, S, part, qt * BR,
                                          qt * BR + BR < N ? qt * BR + BR : N);
            }
          }
        }
      }
    }
  }
}

// Decode's split kernel: split s covers keys [s chunk, min(Nkv, (s + 1) chunk)) in 128-key tiles
// (RG row groups x 4 key splits of 32), each tile clamped to the split's last key.
template <int D>
void sweep_decode() {
  for (int RG : {1, 2}) {
    const Variant v{D, RG, 4, 32};
    check_operand_reads<D>(v);
    for (int nkv : {1, 31, 32, 127, 128, 129, 300, 1000, 4097}) {
      const int tiles = (nkv + 127) / 128;
      for (int S : {1, 2, 3, 7}) {
        if (S > tiles) continue;
        const int chunk = (tiles + S - 1) / S * 128;
        const int splits = (nkv + chunk - 1) / chunk;
        for (int s = 0; s < splits; ++s) {
          const int k_begin = s * chunk;
          const int nk = (nkv < k_begin + chunk ? nkv : k_begin + chunk) - k_begin;
          for (int t = 0; t * 128 < nk; ++t) {
            // The split's keys are a [nk, D] window of the head starting at row k_begin.
            const std::string c = "decode " + std::to_string(D) + " RG=" + std::to_string(RG) +
                                  " Nkv=" + std::to_string(nkv) + " S=" + std::to_string(S) +
                                  " split=" + std::to_string(s);
            check_tile_load<D, false>(v, nk, D, t * 128, true, c);
            check_tile_load<D, true>(v, nk, D, t * 128, true, c);
          }
        }
      }
    }
  }
}

// The grid decode (layout::grid_item) over a sweep of grids, in both orders: every workgroup gets
// an in-range (bh, qt, part) and no two the same one (so all of them are covered); in the
// tile-major order the parts of a query tile are issued one after another on one XCD, and each
// XCD issues its causal query tiles longest first. The head-major order is checked to break that
// last property on the same grids, which is why causal grids take the tile-major order, and which
// shows the check can fail.
void check_grid_items() {
  for (int BH : {1, 3, 8, 16, 24, 96, 100}) {
    for (int nq : {1, 2, 7, 16}) {
      for (int S : {1, 2, 3}) {
        for (bool causal : {false, true}) {
          // order 0 head-major, 1 tile-major, 2 and 3 tile-major in snake order (3 and 32 CUs
          // per XCD).
          for (int order = 0; order < 4; ++order) {
            const int xh = order ? fa::layout::xcd_heads_for(BH, causal) : 0;
            if (order >= 1 && xh == 0) continue;
            const int cus = order == 2 ? 3 : order == 3 ? 32 : 0;
            const int G = nq * BH * S;
            const std::string c = "grid BH=" + std::to_string(BH) + " nq=" + std::to_string(nq) +
                                  " S=" + std::to_string(S) + (causal ? " causal" : "") +
                                  (order == 0 ? " head-major" : " tile-major") +
                                  (cus ? " snake " + std::to_string(cus) : "");
            auto decode = [&](int bid) {
              return fa::layout::grid_item(
                  bid, G, nq, S, causal, xh, cus, [S](int v) { return v / S; },
                  [nq](int v) { return v / nq; }, [xh](int v) { return xh > 0 ? v / xh : 0; },
                  [cus](int v) { return cus > 0 ? v / cus : 0; });
            };
            std::vector<char> seen(static_cast<size_t>(G), 0);
            std::vector<std::vector<int>> issued(fa::layout::kXcds);  // qt per XCD, issue order
            for (int bid = 0; bid < G; ++bid) {
              const auto it = decode(bid);
              if (it.bh < 0 || it.bh >= BH || it.qt < 0 || it.qt >= nq || it.part < 0 ||
                  it.part >= S) {
                fail("grid item out of range: " + c);
              }
              char& s = seen[static_cast<size_t>((it.bh * nq + it.qt) * S + it.part)];
              if (s) fail("grid item issued twice: " + c);
              s = 1;
              if (order >= 1 && it.part + 1 < S) {
                const auto nx = decode(bid + fa::layout::kXcds);
                if (nx.bh != it.bh || nx.qt != it.qt || nx.part != it.part + 1) {
                  fail("parts of a query tile not consecutive on one XCD: " + c);
                }
              }
              if (it.part == 0) issued[bid % fa::layout::kXcds].push_back(it.qt);
              ++g_checks;
            }
            if (!causal) continue;
            bool longest_first = true;
            for (const auto& q : issued) {
              for (size_t i = 1; i < q.size(); ++i) longest_first &= q[i] <= q[i - 1];
            }
            if (order == 1 && !longest_first) fail("tile-major order not longest first: " + c);
            // Snake order: the i-th workgroups of rounds 2r and 2r + 1 share a CU; in full
            // rounds their walks are (longest, shortest) of the pair of rounds.
            if (order >= 2 && S == 1) {
              for (const auto& q : issued) {
                for (size_t r = 0; (r + 2) * cus <= q.size(); r += 2) {
                  for (int i = 0; i + 1 < cus; ++i) {
                    const int a0 = q[r * cus + i], a1 = q[r * cus + i + 1];
                    const int b0 = q[(r + 1) * cus + i], b1 = q[(r + 1) * cus + i + 1];
                    if (a1 > a0 || b1 < b0) fail("snake order rounds not opposed: " + c);
                  }
                }
              }
            }
            if (order == 0 && fa::layout::xcd_heads_for(BH, true) > 1 && nq > 1 && longest_first) {
              fail("head-major order unexpectedly longest first: " + c);
            }
          }
        }
      }
    }
  }
}

}  // namespace

// The rotated walk order (one start per 128-row block, or per group of blocks) keeps results
// independent of the workgroup height: every 32-row wave meets the same key tiles in the same
// order at heights 32, 64 and 128 (the kernel computes a wave's rows from its own tiles only, so
// equal tile sequences give equal bits). A wave's sequence
// is the walk order of its workgroup restricted to the tiles holding a key it can see.
void check_rotation_height_invariance() {
  for (const int groups_lg : {-1, 1, 2}) {
  for (int BC : {32, 64, 128}) {
    for (int N : {32, 96, 128, 224, 512, 640, 1024, 1056, 2048}) {
      for (bool causal : {false, true}) {
        const int n_blocks = (N + fa::layout::kRotRows - 1) / fa::layout::kRotRows;
        for (int r0 = 0; r0 < N; r0 += 32) {
          std::vector<std::vector<int>> seqs;
          for (int BR : {128, 64, 32}) {
            const int qt = r0 / BR;
            auto w = fa::layout::plan_walk(N, BC, BR, qt, causal, 0, [](int x) { return x; });
            fa::layout::rotate_walk(w, N, BC, BR, qt, causal, 0, [](int x) { return x; },
                                    [n_blocks](int x) { return x / n_blocks; }, groups_lg);
            const int wave_end = causal ? (r0 + 32 < N ? r0 + 32 : N) : N;
            std::vector<int> seq;
            for (int t = w.t0; t < w.n_tiles; ++t) {
              const int k = fa::layout::walk_tile(w, t);
              if (k * BC < wave_end) seq.push_back(k);
            }
            seqs.push_back(seq);
            ++g_checks;
          }
          if (seqs[0] != seqs[1] || seqs[0] != seqs[2]) {
            fail("rotated walk differs between heights: BC=" + std::to_string(BC) + " N=" +
                 std::to_string(N) + (causal ? " causal" : "") + " rows " + std::to_string(r0) +
                 " groups_lg " + std::to_string(groups_lg));
          }
        }
      }
    }
  }
  }
}

int main(int argc, char** argv) {
  // Arguments: D,RG,KS,BCW for each stage-4/5 variant of the kernel tables.
  int n = 0;
  for (int i = 1; i < argc; ++i) {
    if (std::string(argv[i]) == "--plant-no-clamp") {
      g_plant_no_clamp = true;
      continue;
    }
    Variant v{};
    if (std::sscanf(argv[i], "%d,%d,%d,%d", &v.D, &v.RG, &v.KS, &v.BCW) != 4) fail(argv[i]);
    if (v.D == 64) sweep_variant<64>(v);
    else if (v.D == 128) sweep_variant<128>(v);
    else fail("unknown head dim");
    ++n;
  }
  sweep_decode<64>();
  sweep_decode<128>();
  check_grid_items();
  check_rotation_height_invariance();
  std::printf("address model: %d variants, decode and the grid decode, %lld checks, all in bounds\n",
              n, g_checks);
  return 0;
}
