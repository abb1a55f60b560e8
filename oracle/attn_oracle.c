/* attn_oracle.c -- fp64 CPU oracle (TEST INFRASTRUCTURE; see attn_oracle.h for who may call it).
 *
 * Two forms of the same function, as in the reference oracle:
 *   direct  (fao_attention_rows / fao_attention): materialise one row's scaled scores, take the
 *           row max, exponentiate, sum, accumulate p*v, divide once
 *           (ref:src/reference/cpu_reference.cpp:47-81);
 *   tiled   (fao_attention_tiled): the online-softmax recurrence of the fused kernels in fp64, with
 *           raw-score running max, the exp2 constant c = scale*log2(e), the alpha / l == 0 guards
 *           and fully-masked causal tiles skipped before any load
 *           (ref:src/reference/cpu_reference.cpp:94-165, ref:include/fa/softmax_math.cuh:25-71).
 * Guards: a row with no visible key gives o = 0 and lse = +inf (ref:include/fa/softmax_math.cuh:54-71).
 */
#include "attn_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static const double kLog2e = 1.4426950408889634;

static size_t row_index(const fao_shape* s, int heads, int b, int h, int n) {
  return (((size_t)b * (size_t)heads + (size_t)h) * (size_t)s->N + (size_t)n) * (size_t)s->D;
}

static int kv_head_of(const fao_shape* s, int h) { return h / (s->H / s->Hkv); }

static double dot(const double* a, const double* b, int d) {
  double acc = 0.0;
  for (int i = 0; i < d; ++i) acc += a[i] * b[i];
  return acc;
}

void fao_attention_rows(const double* q, const double* k, const double* v, const fao_shape* s,
                        int b, int h, int row0, int rows, double* o, double* lse) {
  const int hk = kv_head_of(s, h);
  double* scores = (double*)malloc(sizeof(double) * (size_t)s->N);
  for (int r = 0; r < rows; ++r) {
    const int i = row0 + r;
    const double* qi = q + row_index(s, s->H, b, h, i);
    const int last = s->causal ? i : s->N - 1; /* top-left causal: key j visible iff j <= i */
    double m = -INFINITY;
    for (int j = 0; j < s->N; ++j) {
      const double sc = (j <= last) ? s->scale * dot(qi, k + row_index(s, s->Hkv, b, hk, j), s->D)
                                    : -INFINITY;
      scores[j] = sc;
      if (sc > m) m = sc;
    }
    double* oi = o + (size_t)r * (size_t)s->D;
    memset(oi, 0, sizeof(double) * (size_t)s->D);
    if (m == -INFINITY) { /* no visible key: o = 0, lse = +inf */
      if (lse) lse[r] = INFINITY;
      continue;
    }
    double l = 0.0;
    for (int j = 0; j <= last; ++j) {
      const double p = exp(scores[j] - m);
      const double* vj = v + row_index(s, s->Hkv, b, hk, j);
      l += p;
      for (int d = 0; d < s->D; ++d) oi[d] += p * vj[d];
    }
    for (int d = 0; d < s->D; ++d) oi[d] /= l;
    if (lse) lse[r] = m + log(l); /* scores are already scaled: m + ln l = m_raw*scale + ln l */
  }
  free(scores);
}

void fao_attention(const double* q, const double* k, const double* v, const fao_shape* s,
                   double* o, double* lse) {
  for (int b = 0; b < s->B; ++b) {
    for (int h = 0; h < s->H; ++h) {
      double* ob = o + row_index(s, s->H, b, h, 0);
      double* lb = lse ? lse + ((size_t)b * (size_t)s->H + (size_t)h) * (size_t)s->N : NULL;
      fao_attention_rows(q, k, v, s, b, h, 0, s->N, ob, lb);
    }
  }
}

void fao_attention_tiled(const double* q, const double* k, const double* v, const fao_shape* s,
                         int block_m, int block_n, double* o, double* lse) {
  const double c = s->scale * kLog2e;
  double* m = (double*)malloc(sizeof(double) * (size_t)block_m);
  double* l = (double*)malloc(sizeof(double) * (size_t)block_m);
  double* acc = (double*)malloc(sizeof(double) * (size_t)block_m * (size_t)s->D);
  double* sc = (double*)malloc(sizeof(double) * (size_t)block_n);
  for (int b = 0; b < s->B; ++b) {
    for (int h = 0; h < s->H; ++h) {
      const int hk = kv_head_of(s, h);
      for (int bm = 0; bm < s->N; bm += block_m) {
        const int rows = (block_m < s->N - bm) ? block_m : s->N - bm;
        for (int r = 0; r < rows; ++r) {
          m[r] = -INFINITY;
          l[r] = 0.0;
        }
        memset(acc, 0, sizeof(double) * (size_t)block_m * (size_t)s->D);
        for (int bn = 0; bn < s->N; bn += block_n) {
          if (s->causal && bn > bm + rows - 1) break; /* tile wholly above the diagonal */
          const int cols = (block_n < s->N - bn) ? block_n : s->N - bn;
          for (int r = 0; r < rows; ++r) {
            const int i = bm + r;
            const double* qi = q + row_index(s, s->H, b, h, i);
            double tmax = -INFINITY;
            for (int cj = 0; cj < cols; ++cj) {
              const int j = bn + cj;
              const double raw = (!s->causal || j <= i)
                                     ? dot(qi, k + row_index(s, s->Hkv, b, hk, j), s->D)
                                     : -INFINITY; /* raw units: scale lives in c */
              sc[cj] = raw;
              if (raw > tmax) tmax = raw;
            }
            const double m_old = m[r];
            const double m_new = (tmax > m_old) ? tmax : m_old;
            if (m_new == -INFINITY) continue; /* nothing visible yet: nothing to rescale */
            const double alpha = (m_old == -INFINITY) ? 0.0 : exp2((m_old - m_new) * c);
            double* ar = acc + (size_t)r * (size_t)s->D;
            double rowsum = 0.0;
            for (int d = 0; d < s->D; ++d) ar[d] *= alpha;
            for (int cj = 0; cj < cols; ++cj) {
              const double p = (sc[cj] == -INFINITY) ? 0.0 : exp2((sc[cj] - m_new) * c);
              const double* vj = v + row_index(s, s->Hkv, b, hk, bn + cj);
              rowsum += p;
              for (int d = 0; d < s->D; ++d) ar[d] += p * vj[d];
            }
            l[r] = alpha * l[r] + rowsum;
            m[r] = m_new;
          }
        }
        for (int r = 0; r < rows; ++r) { /* deferred normalisation with the l == 0 guard */
          const int i = bm + r;
          const double inv = (l[r] > 0.0) ? 1.0 / l[r] : 0.0;
          double* oi = o + row_index(s, s->H, b, h, i);
          const double* ar = acc + (size_t)r * (size_t)s->D;
          for (int d = 0; d < s->D; ++d) oi[d] = ar[d] * inv;
          if (lse) {
            lse[((size_t)b * (size_t)s->H + (size_t)h) * (size_t)s->N + (size_t)i] =
                (l[r] > 0.0 && m[r] != -INFINITY) ? m[r] * s->scale + log(l[r]) : INFINITY;
          }
        }
      }
    }
  }
  free(m);
  free(l);
  free(acc);
  free(sc);
}

typedef struct mt_job {
  const double* q;
  const double* k;
  const double* v;
  const fao_shape* s;
  double* o;
  double* lse;
  int first; /* first flat head index b*H + h */
  int count;
} mt_job;

static void* mt_worker(void* arg) {
  const mt_job* j = (const mt_job*)arg;
  for (int bh = j->first; bh < j->first + j->count; ++bh) {
    const int b = bh / j->s->H, h = bh % j->s->H;
    double* ob = j->o + row_index(j->s, j->s->H, b, h, 0);
    double* lb = j->lse ? j->lse + (size_t)bh * (size_t)j->s->N : NULL;
    fao_attention_rows(j->q, j->k, j->v, j->s, b, h, 0, j->s->N, ob, lb);
  }
  return NULL;
}

int fao_attention_mt(const double* q, const double* k, const double* v, const fao_shape* s,
                     double* o, double* lse, int threads) {
  const int heads = s->B * s->H;
  if (threads < 1) threads = 1;
  if (threads > heads) threads = heads;
  pthread_t* tid = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
  mt_job* jobs = (mt_job*)malloc(sizeof(mt_job) * (size_t)threads);
  int next = 0, rc = 0, started = 0;
  for (int t = 0; t < threads; ++t) {
    const int count = heads / threads + (t < heads % threads ? 1 : 0);
    jobs[t] = (mt_job){q, k, v, s, o, lse, next, count};
    next += count;
    if (pthread_create(&tid[t], NULL, mt_worker, &jobs[t]) != 0) {
      rc = -1;
      break;
    }
    ++started;
  }
  for (int t = 0; t < started; ++t) pthread_join(tid[t], NULL);
  free(tid);
  free(jobs);
  return rc;
}
