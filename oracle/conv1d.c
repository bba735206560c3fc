/*
 * TEST INFRASTRUCTURE — CPU oracle, not product code.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this.
 *
 * Plain-C restatement of the reference's CPU path for the causal conv,
 * scripts/cpu_reference.py:40-63 (causal_conv1d_numpy):
 *   out = bias broadcast over [B, D, S]          (cpu_reference.py:56)
 *   for k in 0..W-1: out += w[:, k] * xpad[k : k+S]   (cpu_reference.py:58-62)
 * with xpad = x left-padded by W-1 zeros (cpu_reference.py:54).  Each tap is a
 * separate multiply then add in fp32, in tap order; this file is compiled with
 * -ffp-contract=off so no FMA is formed.
 */
#include <stdint.h>

void oracle_causal_conv1d_f32(const float* x, const float* w, const float* bias, float* out,
                              int64_t B, int64_t D, int64_t S, int32_t W) {
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t d = 0; d < D; ++d) {
      const float* xr = x + (b * D + d) * S;
      float* orow = out + (b * D + d) * S;
      const float* wr = w + d * W;
      const float bd = bias ? bias[d] : 0.0f;
      for (int64_t t = 0; t < S; ++t) orow[t] = bd;
      for (int32_t k = 0; k < W; ++k) {
        const float wk = wr[k];
        const int64_t shift = (int64_t)(W - 1 - k); /* xpad[k + t] = x[t - shift] */
        for (int64_t t = shift; t < S; ++t) {
          const float prod = wk * xr[t - shift];
          orow[t] = orow[t] + prod;
        }
      }
    }
  }
}
