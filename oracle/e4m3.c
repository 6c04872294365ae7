/* CPU oracle (TEST INFRASTRUCTURE ONLY): OCP e4m3fn encoder by nearest-value search over the 127 non-negative finite
 * code values (ties -> the code with an even mantissa), independent of the bit-arithmetic encoders of the kernels and
 * of oracle/spmla_ref.py. Magnitudes at or beyond the midpoint 464 between 448 and the (absent) next value 480 encode
 * as NaN (0x7f) except exactly 464, which ties to 448; inf / NaN -> NaN. Sign copied (so -0 -> 0x80).
 * Reference conversions this restates: torch / Triton float8_e4m3fn RNE casts at
 * dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:263-266 and dotsnote/training/finetune/student.py:87. */
#include <math.h>
#include <stdint.h>
#include <string.h>

static double g_val[127];
static int g_init = 0;

static void init_table(void) {
  for (int c = 0; c < 127; ++c) {
    int e = (c >> 3) & 15, m = c & 7;
    g_val[c] = e == 0 ? m * ldexp(1.0, -9) : ldexp(1.0 + m / 8.0, e - 7);
  }
  g_init = 1;
}

uint8_t oracle_e4m3_encode(float x) {
  if (!g_init) init_table();
  uint32_t u;
  memcpy(&u, &x, 4);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  double a = fabs((double)x);
  if (isnan(x) || isinf(x)) return sign | 0x7f;
  if (a > 464.0) return sign | 0x7f;
  /* binary search for the largest code value <= a */
  int lo = 0, hi = 126;
  while (lo < hi) {
    int mid = (lo + hi + 1) / 2;
    if (g_val[mid] <= a) lo = mid; else hi = mid - 1;
  }
  int c = lo;
  if (c < 126) {
    double d0 = a - g_val[c], d1 = g_val[c + 1] - a;
    if (d1 < d0 || (d1 == d0 && ((c + 1) & 1) == 0)) c = c + 1;
  }
  return sign | (uint8_t)c;
}

void oracle_e4m3_encode_n(const float* x, uint8_t* out, long long n) {
  for (long long i = 0; i < n; ++i) out[i] = oracle_e4m3_encode(x[i]);
}

/* encode the fp32 bit patterns start, start + 1, ..., start + n - 1 */
void oracle_e4m3_encode_bits(uint32_t start, long long n, uint8_t* out) {
  for (long long i = 0; i < n; ++i) {
    uint32_t b = start + (uint32_t)i;
    float f;
    memcpy(&f, &b, 4);
    out[i] = oracle_e4m3_encode(f);
  }
}
