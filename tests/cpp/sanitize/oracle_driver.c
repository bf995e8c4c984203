/* Driver for the ASan/UBSan build of the oracle's C restatement
 * (oracle/attn_ref.c): ragged texts, GQA, causal and windowed masks, each
 * row checked against a direct two-pass softmax in double precision. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

int inl_ref_attn_f32(int n_texts, const int32_t* cu, int hq, int hkv, int d, int causal, int window, float scale,
                     const float* q, const float* k, const float* v, float* out);

static uint64_t state = 88172645463325252ull;
static float uni(void) {
  state ^= state << 13; state ^= state >> 7; state ^= state << 17;
  return (float)((state >> 11) * (1.0 / 9007199254740992.0)) * 2.f - 1.f;
}

int main(void) {
  int failures = 0, cases = 0;
  const int lens[] = {0, 1, 5, 16, 17, 33, 70};
  for (int c = 0; c < 24; ++c) {
    const int n = 1 + c % 5, hkv = 1 + c % 2, hq = hkv * (1 + c % 3), d = 8 * (1 + c % 4);
    const int causal = c % 2, window = (c % 3 == 0) ? -1 : (c % 7);
    int32_t cu[8];
    cu[0] = 0;
    for (int b = 0; b < n; ++b) cu[b + 1] = cu[b] + lens[(c + 3 * b) % 7];
    const int N = cu[n];
    float* q = malloc(sizeof(float) * (N * hq * d + 1));
    float* k = malloc(sizeof(float) * (N * hkv * d + 1));
    float* v = malloc(sizeof(float) * (N * hkv * d + 1));
    float* o = malloc(sizeof(float) * (N * hq * d + 1));
    for (int i = 0; i < N * hq * d; ++i) q[i] = uni();
    for (int i = 0; i < N * hkv * d; ++i) { k[i] = uni(); v[i] = uni(); }
    if (inl_ref_attn_f32(n, cu, hq, hkv, d, causal, window, 0.3f, q, k, v, o) != 0) { ++failures; continue; }
    for (int b = 0; b < n; ++b)
      for (int i = 0; i < cu[b + 1] - cu[b]; ++i)
        for (int h = 0; h < hq; ++h) {
          const int kh = h / (hq / hkv), T = cu[b + 1] - cu[b];
          double mx = -1e300, l = 0, acc[32] = {0};
          for (int pass = 0; pass < 2; ++pass)
            for (int j = 0; j < T; ++j) {
              if ((causal && j > i) || (window >= 0 && abs(i - j) > window)) continue;
              double s = 0;
              for (int e = 0; e < d; ++e)
                s += (double)q[((cu[b] + i) * hq + h) * d + e] * k[((cu[b] + j) * hkv + kh) * d + e];
              s *= 0.3;
              if (pass == 0) { if (s > mx) mx = s; continue; }
              const double p = exp(s - mx);
              l += p;
              for (int e = 0; e < d; ++e) acc[e] += p * v[((cu[b] + j) * hkv + kh) * d + e];
            }
          for (int e = 0; e < d; ++e) {
            const double want = l > 0 ? acc[e] / l : 0.0;
            ++cases;
            if (fabs(want - o[((cu[b] + i) * hq + h) * d + e]) > 1e-5) ++failures;
          }
        }
    free(q); free(k); free(v); free(o);
  }
  /* refusals */
  ++cases;
  if (inl_ref_attn_f32(1, NULL, 3, 2, 8, 0, -1, 1.f, NULL, NULL, NULL, NULL) != -1) ++failures;
  printf("%d cases, %d failures\n", cases, failures);
  return failures ? 1 : 0;
}
