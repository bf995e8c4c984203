/*
 * attn_ref.c - f32 CPU restatement of the reference's CPU attention path.
 * TEST INFRASTRUCTURE ONLY: used by tests (as a second, independent oracle
 * implementation) and by bench.py's cpu_baseline leg (as the timed CPU
 * baseline). Never linked into the product library.
 *
 * It follows crates/inl-core/src/attention.rs:282-315 (`cpu_flash`): each
 * text is attended on its real tokens only, with candle's CPU flash
 * attention - an online softmax over key blocks with a running max and sum,
 * in f32 - and the packed generalisation the encoder forms need
 * (bidirectional, inclusive-radius windows: gemma2.rs:515,
 * modernbert.rs:607). GQA: query head h reads KV head h / (hq / hkv).
 *
 * Layout: q [N, hq, d], k/v [N, hkv, d], out [N, hq, d], row-major f32,
 * texts at cu[b]..cu[b+1]. Parallel over (text, head, query block) with
 * OpenMP.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define KEY_BLOCK 64
#define MAX_D 512

static void attend_row(const float* qi, const float* kbase, const float* vbase,
                       int64_t kv_stride, int d, int lo, int hi, float scale,
                       float* out) {
  float acc[MAX_D];
  float s[KEY_BLOCK];
  float m = -INFINITY, l = 0.f;
  for (int e = 0; e < d; ++e) acc[e] = 0.f;
  for (int j0 = lo; j0 < hi; j0 += KEY_BLOCK) {
    const int j1 = j0 + KEY_BLOCK < hi ? j0 + KEY_BLOCK : hi;
    float bm = -INFINITY;
    for (int j = j0; j < j1; ++j) {
      const float* kj = kbase + (int64_t)j * kv_stride;
      /* eight interleaved partial sums in a fixed order, so the compiler
       * can use 8-wide vector FMAs without reassociating (no fast-math) */
      float part[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      int e = 0;
      for (; e + 8 <= d; e += 8)
        for (int u = 0; u < 8; ++u) part[u] += qi[e + u] * kj[e + u];
      for (; e < d; ++e) part[e & 7] += qi[e] * kj[e];
      float dot = ((part[0] + part[4]) + (part[2] + part[6])) + ((part[1] + part[5]) + (part[3] + part[7]));
      dot *= scale;
      s[j - j0] = dot;
      if (dot > bm) bm = dot;
    }
    const float mn = bm > m ? bm : m;
    const float alpha = expf(m - mn); /* m = -inf on the first block -> 0 */
    l *= alpha;
    for (int e = 0; e < d; ++e) acc[e] *= alpha;
    for (int j = j0; j < j1; ++j) {
      const float p = expf(s[j - j0] - mn);
      const float* vj = vbase + (int64_t)j * kv_stride;
      l += p;
      for (int e = 0; e < d; ++e) acc[e] += p * vj[e];
    }
    m = mn;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  for (int e = 0; e < d; ++e) out[e] = acc[e] * inv;
}

/* Returns 0 on success, -1 on a bad argument. */
int inl_ref_attn_f32(int n_texts, const int32_t* cu, int hq, int hkv, int d,
                     int causal, int window, float scale, const float* q,
                     const float* k, const float* v, float* out) {
  if (n_texts < 0 || hq <= 0 || hkv <= 0 || hq % hkv || d <= 0 || d > MAX_D) return -1;
  const int group = hq / hkv;
  const int QB = 16; /* query rows per parallel work unit */
  /* flatten (text, head, query block) into one parallel loop */
  int64_t units = 0;
  for (int b = 0; b < n_texts; ++b) units += (int64_t)hq * ((cu[b + 1] - cu[b] + QB - 1) / QB);
  int64_t* starts = (int64_t*)malloc(sizeof(int64_t) * (n_texts + 1));
  if (!starts) return -1;
  starts[0] = 0;
  for (int b = 0; b < n_texts; ++b)
    starts[b + 1] = starts[b] + (int64_t)hq * ((cu[b + 1] - cu[b] + QB - 1) / QB);
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t u = 0; u < units; ++u) {
    int b = 0;
    { /* binary search for the text */
      int lo = 0, hi = n_texts - 1;
      while (lo < hi) {
        int mid = (lo + hi + 1) / 2;
        if (starts[mid] <= u) lo = mid; else hi = mid - 1;
      }
      b = lo;
    }
    const int T = cu[b + 1] - cu[b];
    const int nqb = (T + QB - 1) / QB;
    const int64_t r = u - starts[b];
    const int h = (int)(r / nqb);
    const int qb = (int)(r % nqb);
    const int kvh = h / group;
    const float* kb = k + ((int64_t)cu[b] * hkv + kvh) * d;
    const float* vb = v + ((int64_t)cu[b] * hkv + kvh) * d;
    for (int i = qb * QB; i < T && i < (qb + 1) * QB; ++i) {
      int lo = 0, hi = causal ? i + 1 : T;
      if (window >= 0) {
        if (i - window > lo) lo = i - window;
        if (i + window + 1 < hi) hi = i + window + 1;
      }
      const int64_t row = (int64_t)cu[b] + i;
      attend_row(q + (row * hq + h) * d, kb, vb, (int64_t)hkv * d, d, lo, hi, scale,
                 out + (row * hq + h) * d);
    }
  }
  free(starts);
  return 0;
}

int inl_ref_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}
