/* Compares hale_expf (hale-token_amd/csrc/glibc_expf.h, the device exp used
 * by SiLU and softmax) with the host glibc expf on every non-NaN float.
 * Prints the number of mismatches.  Built and run by tests/test_expf.py. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "glibc_expf.h"

int main(void) {
  unsigned long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (long long hi = 0; hi < 65536; hi++) {
    for (uint32_t lo = 0; lo < 65536; lo++) {
      uint32_t u = ((uint32_t)hi << 16) | lo;
      float x, a, b;
      memcpy(&x, &u, 4);
      if (isnan(x)) continue;
      a = expf(x);
      b = hale_expf(x);
      if (memcmp(&a, &b, 4) != 0) bad++;
    }
  }
  printf("%llu\n", bad);
  return 0;
}
