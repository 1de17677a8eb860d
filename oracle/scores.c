/* Oracle (test infrastructure only): the QSA block scores of
 * reference/model.py:297-298,
 *     s[b, q, j] = sum_h relu(q[b, q, h, :] . k[b, j, :]) / sqrt(d),
 * restated with the exact float32 summation orders the reference's CPU path
 * (torch's einsum on its BLAS) takes, as pinned bit for bit by the golden
 * score vectors of tests/golden (cfg3, cfg3b: one query row; cfg5: 128 rows):
 *   one query row (S == 1): 16 partial sums, partial m accumulating elements
 *     m, m + 16, ..., m + 112 by fused multiply-add in that order; partials m,
 *     m + 4, m + 8, m + 12 added in that order into c_(m mod 4); the dot
 *     product is (c0 + c1) + (c2 + c3);
 *   several rows (S > 1): one fused multiply-add chain over d = 0 .. 127;
 * then ((relu(D_0) + relu(D_1)) + relu(D_2)) + relu(D_3) over the heads and a
 * float division by sqrt(128) rounded to float. Compile without contraction
 * (-ffp-contract=off): every add is rounded on its own. */
#include <math.h>

static float dot16(const float* a, const float* b) {
  float p[16];
  for (int m = 0; m < 16; ++m) p[m] = 0.f;
  for (int d = 0; d < 128; ++d) p[d & 15] = fmaf(a[d], b[d], p[d & 15]);
  float c[4];
  for (int l = 0; l < 4; ++l) c[l] = ((p[l] + p[4 + l]) + p[8 + l]) + p[12 + l];
  return (c[0] + c[1]) + (c[2] + c[3]);
}

static float dot_seq(const float* a, const float* b) {
  float s = 0.f;
  for (int d = 0; d < 128; ++d) s = fmaf(a[d], b[d], s);
  return s;
}

/* q [B, S, H, 128], k [B, N, 128], out [B, S, N], all float32, contiguous */
void oracle_block_scores(const float* q, const float* k, int B, int S, int H, int N, float* out) {
  const float sq = (float)sqrt(128.0);
  for (int b = 0; b < B; ++b)
    for (int s = 0; s < S; ++s)
      for (int j = 0; j < N; ++j) {
        float sc = 0.f;
        for (int h = 0; h < H; ++h) {
          const float* a = q + (((long)b * S + s) * H + h) * 128;
          const float* kb = k + ((long)b * N + j) * 128;
          const float dv = S == 1 ? dot16(a, kb) : dot_seq(a, kb);
          sc = sc + (dv > 0.f ? dv : 0.f);
        }
        out[((long)b * S + s) * N + j] = sc / sq;
      }
}
