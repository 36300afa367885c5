/* Compares the oracle's f32->f16 conversion with the x86 F16C instruction
 * (vcvtps2ph, round to nearest even) on every non-NaN float bit pattern.
 * Prints the number of mismatches.  Built and run by tests/test_oracle.py. */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void orc_f32_to_f16_range(uint32_t lo, size_t n, uint16_t *out);

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
  printf("%llu\n", bad);
  free(ours);
  return 0;
}
