/* attn_oracle.h -- fp64 CPU oracle for the fused SDPA forward.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker (or the timed CPU baseline),
 * never as the thing measured or shipped. The product path (libfa_hip.so, fused_attn._C) never
 * links or calls it.
 *
 * A plain-C restatement of the reference's fp64 CPU oracle:
 *   fao_attention_rows   <- fa::ref::attention_rows   (ref:src/reference/cpu_reference.cpp:47-81)
 *   fao_attention        <- fa::ref::attention        (ref:src/reference/cpu_reference.cpp:83-92)
 *   fao_attention_tiled  <- fa::ref::attention_tiled  (ref:src/reference/cpu_reference.cpp:94-165)
 *   fao_attention_mt     the same direct form, heads spread over POSIX threads (the multi-core CPU
 *                        baseline; bitwise identical to fao_attention because every head is
 *                        computed by the same scalar code in the same order).
 * Layouts follow ref:include/fa/attention.cuh:38-45: q/o [B,H,N,D], k/v [B,Hkv,N,D], lse [B,H,N],
 * all contiguous, D fastest. Causal is top-left (key j visible to query i iff j <= i); query head h
 * reads kv head h / (H / Hkv).
 *
 * Pinned by tests/test_oracle_cpu.py against: the reference's own compiled oracle (golden vectors
 * in tests/golden/, written by oracle/_ref from the reference sources), the 2x2 closed form of
 * ref:src/reference/test_cpu_reference.cpp:39-67, torch SDPA MATH fp64, tiled == direct for odd
 * tilings, scale folding and sum_j exp(s_ij - lse_i) == 1.
 */
#ifndef FA_ATTN_ORACLE_H_
#define FA_ATTN_ORACLE_H_

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fao_shape {
  int B;
  int H;
  int Hkv;
  int N;
  int D;
  double scale;
  int causal;
} fao_shape;

void fao_attention_rows(const double* q, const double* k, const double* v, const fao_shape* s,
                        int b, int h, int row0, int rows, double* o, double* lse);
void fao_attention(const double* q, const double* k, const double* v, const fao_shape* s,
                   double* o, double* lse);
void fao_attention_tiled(const double* q, const double* k, const double* v, const fao_shape* s,
                         int block_m, int block_n, double* o, double* lse);
/* Direct form over `threads` POSIX threads, heads partitioned statically. Returns 0 on success. */
int fao_attention_mt(const double* q, const double* k, const double* v, const fao_shape* s,
                     double* o, double* lse, int threads);

#ifdef __cplusplus
}
#endif

#endif /* FA_ATTN_ORACLE_H_ */
