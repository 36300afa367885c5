/* Compares the oracle's f32->f16 conversion with the x86 F16C instruction
 * (vcvtps2ph, round to nearest even) on every non-NaN float bit pattern,
 * and its f16->f32 conversion with vcvtph2ps on every half bit pattern, NaNs
 * included, bit for bit.  Prints the two mismatch counts.  Built and run by
 * tests/test_oracle.py. */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void orc_f32_to_f16_range(uint32_t lo, size_t n, uint16_t *out);
float orc_f16_to_f32(uint16_t h);

int main(void) {
  const size_t chunk = (size_t)1 << 24;
  uint16_t *ours = malloc(chunk * 2);
  unsigned long long bad = 0;
  for (uint64_t lo = 0; lo < (1ull << 32); lo += chunk) {
    orc_f32_to_f16_range((uint32_t)lo, chunk, ours);
    for (size_t i = 0; i < chunk; i += 8) {
      uint32_t bits[8];
      for (int j = 0; j < 8; j++) bits[j] = (uint32_t)(lo + i + j);
      __m256 v;
      memcpy(&v, bits, 32);
      __m128i h = _mm256_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT);
      uint16_t ref[8];
      memcpy(ref, &h, 16);
      for (int j = 0; j < 8; j++) {
        float f;
        memcpy(&f, &bits[j], 4);
        if (!isnan(f) && ref[j] != ours[i + j]) bad++;
      }
    }
  }
  unsigned long long bad_up = 0;
  for (uint32_t h0 = 0; h0 < 65536; h0 += 8) {
    uint16_t hs[8];
    for (int j = 0; j < 8; j++) hs[j] = (uint16_t)(h0 + j);
    __m128i hv;
    memcpy(&hv, hs, 16);
    __m256 f = _mm256_cvtph_ps(hv);
    uint32_t ref[8];
    memcpy(ref, &f, 32);
    for (int j = 0; j < 8; j++) {
      float o = orc_f16_to_f32(hs[j]);
      uint32_t ob;
      memcpy(&ob, &o, 4);
      if (ob != ref[j]) bad_up++;
    }
  }
  printf("%llu %llu\n", bad, bad_up);
  free(ours);
  return 0;
}
