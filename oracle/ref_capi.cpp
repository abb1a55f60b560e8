// ref_capi.cpp -- C entry points over the REFERENCE's own fp64 CPU oracle.
//
// TEST INFRASTRUCTURE. Compiled by oracle/Makefile together with the reference's unmodified
// source file ref:src/reference/cpu_reference.cpp (read in place from /root/reference; nothing is
// copied) into oracle/_ref/libfa_ref.so. Used only to (a) write the golden vectors under
// tests/golden/ and (b) serve as bench.py's "reference" CPU baseline. This file is original glue:
// it builds the reference's fa::ref::Shape (ref:src/reference/cpu_reference.h:21-29) from plain
// ints and forwards to
//   fa::ref::attention       (ref:src/reference/cpu_reference.h:42-43)
//   fa::ref::attention_rows  (ref:src/reference/cpu_reference.h:38-39)
//   fa::ref::attention_tiled (ref:src/reference/cpu_reference.h:49-50)
// The threaded entry runs the reference's attention_rows for disjoint heads on std::threads
// (the reference itself is single-threaded; each head is computed by its unmodified code).
#include <cstddef>
#include <thread>
#include <vector>

#include "cpu_reference.h"

namespace {

fa::ref::Shape make_shape(int B, int H, int Hkv, int N, int D, double scale, int causal) {
  fa::ref::Shape s;
  s.B = B;
  s.H = H;
  s.Hkv = Hkv;
  s.N = N;
  s.D = D;
  s.scale = scale;
  s.causal = causal != 0;
  return s;
}

}  // namespace

extern "C" {

void faref_attention(const double* q, const double* k, const double* v, int B, int H, int Hkv,
                     int N, int D, double scale, int causal, double* o, double* lse) {
  fa::ref::attention(q, k, v, make_shape(B, H, Hkv, N, D, scale, causal), o, lse);
}

void faref_attention_rows(const double* q, const double* k, const double* v, int B, int H,
                          int Hkv, int N, int D, double scale, int causal, int b, int h, int row0,
                          int rows, double* o, double* lse) {
  fa::ref::attention_rows(q, k, v, make_shape(B, H, Hkv, N, D, scale, causal), b, h, row0, rows, o,
                          lse);
}

void faref_attention_tiled(const double* q, const double* k, const double* v, int B, int H,
                           int Hkv, int N, int D, double scale, int causal, int block_m,
                           int block_n, double* o, double* lse) {
  fa::ref::attention_tiled(q, k, v, make_shape(B, H, Hkv, N, D, scale, causal), block_m, block_n,
                           o, lse);
}

// Heads [head0, head0 + nheads) of the flattened B*H axis, over `threads` std::threads.
// o / lse point at the start of head0's slice (nheads*N*D and nheads*N elements).
void faref_attention_heads_mt(const double* q, const double* k, const double* v, int B, int H,
                              int Hkv, int N, int D, double scale, int causal, int head0,
                              int nheads, double* o, double* lse, int threads) {
  const fa::ref::Shape s = make_shape(B, H, Hkv, N, D, scale, causal);
  if (threads < 1) threads = 1;
  if (threads > nheads) threads = nheads;
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; ++t) {
    pool.emplace_back([&, t] {
      for (int i = t; i < nheads; i += threads) {
        const int bh = head0 + i;
        const std::size_t off = static_cast<std::size_t>(i) * N;
        fa::ref::attention_rows(q, k, v, s, bh / H, bh % H, 0, N, o + off * D,
                                lse ? lse + off : nullptr);
      }
    });
  }
  for (std::thread& th : pool) th.join();
}

}  // extern "C"
