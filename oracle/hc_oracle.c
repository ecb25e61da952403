/*
 * C restatement of the CPU-heavy parts of the oracle.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ as a second implementation and by
 * bench.py's cpu_baseline leg.  Never linked into the product.
 *
 *   hco_decode_attention  softmax(scale q K^T) V per (row, query), natural
 *                         layout K/V, fp32 accumulation, split into token
 *                         chunks merged with the usual (max, sum) rescaling.
 *                         Follows flash_attn_with_kvcache's contract at
 *                         heterocache/llama_model.py:382-389.
 *   hco_topk_select       top-cap positions of a score row under the
 *                         (-score, index) order, returned ascending
 *                         (heterocache/cache_utils.py:831-851).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define D 128

static inline float bf16_to_f32(uint16_t x) {
  uint32_t u = (uint32_t)x << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline float load_elem(const void* base, int dtype, int64_t i) {
  if (dtype == 2) return bf16_to_f32(((const uint16_t*)base)[i]);
  return ((const float*)base)[i];
}

int hco_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void hco_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* dtype: 0 = fp32, 2 = bf16.  q: [rows, G, D]; K/V token t of row r at
 * (row_off[r] + t) * D.  out: [rows, G, D] fp32. */
void hco_decode_attention(int dtype, const void* q, const void* k, const void* v, const int64_t* row_off,
                          const int32_t* row_len, int rows, int G, float scale, int chunk, float* out) {
  if (chunk <= 0) chunk = 4096;
  int64_t* first = (int64_t*)malloc(sizeof(int64_t) * (rows + 1));
  first[0] = 0;
  for (int r = 0; r < rows; ++r) first[r + 1] = first[r] + (row_len[r] + chunk - 1) / chunk;
  const int64_t nparts = first[rows];
  float* pm = (float*)malloc(sizeof(float) * (size_t)(nparts > 0 ? nparts : 1) * G);
  float* pl = (float*)malloc(sizeof(float) * (size_t)(nparts > 0 ? nparts : 1) * G);
  float* po = (float*)malloc(sizeof(float) * (size_t)(nparts > 0 ? nparts : 1) * G * D);

#pragma omp parallel for schedule(dynamic)
  for (int64_t p = 0; p < nparts; ++p) {
    int r = 0;
    while (first[r + 1] <= p) ++r;
    const int64_t c = p - first[r];
    const int t0 = (int)(c * chunk);
    const int t1 = (int)((t0 + chunk < row_len[r]) ? t0 + chunk : row_len[r]);
    float qf[16][D];
    float m[16], l[16], o[16][D];
    for (int g = 0; g < G; ++g) {
      for (int d = 0; d < D; ++d) qf[g][d] = load_elem(q, dtype, ((int64_t)r * G + g) * D + d);
      m[g] = -INFINITY;
      l[g] = 0.f;
      memset(o[g], 0, sizeof(o[g]));
    }
    float kf[D], vf[D];
    for (int t = t0; t < t1; ++t) {
      const int64_t base = (row_off[r] + t) * D;
      for (int d = 0; d < D; ++d) {
        kf[d] = load_elem(k, dtype, base + d);
        vf[d] = load_elem(v, dtype, base + d);
      }
      for (int g = 0; g < G; ++g) {
        float s = 0.f;
        for (int d = 0; d < D; ++d) s += qf[g][d] * kf[d];
        s *= scale;
        if (s > m[g]) {
          const float a = expf(m[g] - s);
          l[g] *= a;
          for (int d = 0; d < D; ++d) o[g][d] *= a;
          m[g] = s;
        }
        const float pr = expf(s - m[g]);
        l[g] += pr;
        for (int d = 0; d < D; ++d) o[g][d] += pr * vf[d];
      }
    }
    for (int g = 0; g < G; ++g) {
      pm[p * G + g] = m[g];
      pl[p * G + g] = l[g];
      memcpy(po + (p * G + g) * D, o[g], sizeof(o[g]));
    }
  }

  for (int r = 0; r < rows; ++r) {
    for (int g = 0; g < G; ++g) {
      float* dst = out + ((int64_t)r * G + g) * D;
      memset(dst, 0, sizeof(float) * D);
      if (first[r + 1] == first[r]) continue;
      float M = -INFINITY;
      for (int64_t p = first[r]; p < first[r + 1]; ++p) M = fmaxf(M, pm[p * G + g]);
      float L = 0.f;
      for (int64_t p = first[r]; p < first[r + 1]; ++p) {
        const float f = expf(pm[p * G + g] - M);
        L += f * pl[p * G + g];
        for (int d = 0; d < D; ++d) dst[d] += f * po[(p * G + g) * D + d];
      }
      for (int d = 0; d < D; ++d) dst[d] /= L;
    }
  }
  free(first);
  free(pm);
  free(pl);
  free(po);
}

typedef struct {
  float s;
  int32_t i;
} hco_pair;

static int cmp_rank(const void* a, const void* b) {
  const hco_pair* x = (const hco_pair*)a;
  const hco_pair* y = (const hco_pair*)b;
  if (x->s > y->s) return -1;
  if (x->s < y->s) return 1;
  return (x->i > y->i) - (x->i < y->i);
}

static int cmp_int(const void* a, const void* b) {
  const int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
  return (x > y) - (x < y);
}

/* Ascending positions of the top-`cap` scores (ties: lower index first). */
int hco_topk_select(const float* scores, int L, int cap, int32_t* out) {
  if (cap > L) cap = L;
  if (cap <= 0) return 0;
  hco_pair* p = (hco_pair*)malloc(sizeof(hco_pair) * (size_t)L);
  for (int i = 0; i < L; ++i) {
    p[i].s = scores[i];
    p[i].i = i;
  }
  qsort(p, (size_t)L, sizeof(hco_pair), cmp_rank);
  for (int i = 0; i < cap; ++i) out[i] = p[i].i;
  free(p);
  qsort(out, (size_t)cap, sizeof(int32_t), cmp_int);
  return cap;
}
