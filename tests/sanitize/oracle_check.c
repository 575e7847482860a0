/* The CPU oracle (oracle/sde_oracle.c) under AddressSanitizer and
 * UndefinedBehaviorSanitizer (TEST INFRASTRUCTURE; built by this folder's
 * Makefile, run by tests/test_sanitize.py).  Every buffer is allocated at
 * its exact size, so a read or write past a pool, table, q or output row
 * is reported.  Random shapes and fragmented block tables; checks that
 * hold whatever the arithmetic's rounding:
 *   - fp16 -> fp32 -> fp16 is the identity on all 65536 bit patterns (NaNs
 *     stay NaN);
 *   - append then gather returns the fp16 rounding of what was appended;
 *   - the tiled fp32 attention is within 2e-5 (relative to max |V|) of the
 *     fp64 one, and a one-key context returns that key's V row;
 *   - the GEMV is within fp32 rounding of an fp64 sum. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

uint16_t oracle_f32_to_f16(float f);
float oracle_f16_to_f32(uint16_t h);
void oracle_kv_append(uint16_t* pool, const int32_t* table, int kv_dim, int bs, const float* k,
                      const float* v, int pos_base, int n);
void oracle_kv_gather(const uint16_t* pool, const int32_t* table, int kv_dim, int bs, int pos,
                      int n, float* k, float* v);
int oracle_paged_attention(const float* q, float* out, double* out_f64, const uint16_t* pool,
                           const int32_t* table, int kv_dim, int bs, int nh, int nkv, int dph,
                           int pos_base, int M, int mode, int n_threads);
void oracle_matvec(const float* x, const uint16_t* W, float* out, int d_in, int d_out,
                   int n_rows, int accumulate);

static uint64_t g_state = 0x243F6A8885A308D3ull;
static uint64_t next_u64(void) {
  g_state ^= g_state >> 12;
  g_state ^= g_state << 25;
  g_state ^= g_state >> 27;
  return g_state * 0x2545F4914F6CDD1Dull;
}
static int rnd(int n) { return (int)(next_u64() % (uint64_t)n); }
static float frnd(void) { return (float)((double)(next_u64() >> 11) / 9007199254740992.0 * 2 - 1); }

static int g_fail = 0;
#define CHECK(c, ...)                                    \
  do {                                                   \
    if (!(c) && ++g_fail <= 20) {                        \
      fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      fprintf(stderr, __VA_ARGS__);                      \
      fprintf(stderr, "\n");                             \
    }                                                    \
  } while (0)

static void* xmalloc(size_t n) {
  void* p = malloc(n ? n : 1);
  if (!p) {
    fprintf(stderr, "out of memory\n");
    exit(2);
  }
  return p;
}

static void check_f16(void) {
  for (uint32_t h = 0; h < 65536u; h++) {
    const float f = oracle_f16_to_f32((uint16_t)h);
    const uint16_t back = oracle_f32_to_f16(f);
    const int nan = (h & 0x7C00u) == 0x7C00u && (h & 0x03FFu) != 0;
    if (nan)
      CHECK(isnan(f) && (back & 0x7C00u) == 0x7C00u && (back & 0x03FFu) != 0, "nan %04x", h);
    else
      CHECK(back == h, "f16 %04x -> %a -> %04x", h, (double)f, back);
  }
}

static void check_case(int it) {
  const int dph = (rnd(2) ? 64 : 128) >> rnd(2);
  const int nkv = 1 << rnd(3), G = 1 << rnd(3), nh = nkv * G;
  const int kv_dim = nkv * dph, bs = 1 + rnd(32), max_blocks = 1 + rnd(12);
  const int n_layers = 1 + rnd(3);
  const int pool_blocks = n_layers * max_blocks + rnd(4);
  const size_t pool_n = (size_t)pool_blocks * 2 * bs * kv_dim;
  uint16_t* pool = xmalloc(pool_n * 2);
  memset(pool, 0, pool_n * 2);
  /* layer tables: disjoint physical blocks in a shuffled order */
  int32_t* perm = xmalloc(sizeof(int32_t) * pool_blocks);
  for (int i = 0; i < pool_blocks; i++) perm[i] = i;
  for (int i = pool_blocks - 1; i > 0; i--) {
    const int j = rnd(i + 1);
    const int32_t t = perm[i];
    perm[i] = perm[j];
    perm[j] = t;
  }
  const int layer = rnd(n_layers);
  const int32_t* table = perm + (size_t)layer * max_blocks; /* exactly max_blocks entries used */
  const int cap = max_blocks * bs;
  const int len = 1 + rnd(cap);
  float* k = xmalloc(sizeof(float) * (size_t)len * kv_dim);
  float* v = xmalloc(sizeof(float) * (size_t)len * kv_dim);
  float vmax = 0.f;
  for (size_t i = 0; i < (size_t)len * kv_dim; i++) {
    k[i] = 2.f * frnd();
    v[i] = frnd();
    if (fabsf(v[i]) > vmax) vmax = fabsf(v[i]);
  }
  /* append in two pieces, as a prefill and a window */
  const int cut = rnd(len + 1);
  oracle_kv_append(pool, table, kv_dim, bs, k, v, 0, cut);
  oracle_kv_append(pool, table, kv_dim, bs, k + (size_t)cut * kv_dim, v + (size_t)cut * kv_dim,
                   cut, len - cut);
  float* kg = xmalloc(sizeof(float) * (size_t)len * kv_dim);
  float* vg = xmalloc(sizeof(float) * (size_t)len * kv_dim);
  oracle_kv_gather(pool, table, kv_dim, bs, 0, len, kg, vg);
  for (size_t i = 0; i < (size_t)len * kv_dim; i++) {
    CHECK(kg[i] == oracle_f16_to_f32(oracle_f32_to_f16(k[i])), "case %d: K gather %zu", it, i);
    CHECK(vg[i] == oracle_f16_to_f32(oracle_f32_to_f16(v[i])), "case %d: V gather %zu", it, i);
  }
  /* a window of M queries ending at len */
  const int M = 1 + rnd(len < 8 ? len : 8);
  const int pos_base = len - M;
  const size_t qn = (size_t)M * nh * dph;
  float* q = xmalloc(sizeof(float) * qn);
  float* out = xmalloc(sizeof(float) * qn);
  double* ref = xmalloc(sizeof(double) * qn);
  for (size_t i = 0; i < qn; i++) q[i] = frnd();
  oracle_paged_attention(q, out, NULL, pool, table, kv_dim, bs, nh, nkv, dph, pos_base, M, 0, 2);
  oracle_paged_attention(q, NULL, ref, pool, table, kv_dim, bs, nh, nkv, dph, pos_base, M, 1, 2);
  for (size_t i = 0; i < qn; i++)
    CHECK(fabs((double)out[i] - ref[i]) <= 2e-5 * (vmax > 1e-6f ? vmax : 1.f) + 1e-7,
          "case %d: attention %zu: %g vs %g", it, i, (double)out[i], ref[i]);
  if (pos_base == 0) { /* the first query sees one key: its V row */
    for (int h = 0; h < nh; h++)
      for (int e = 0; e < dph; e++)
        CHECK(ref[(size_t)h * dph + e] == (double)vg[(size_t)(h / G) * dph + e],
              "case %d: one-key attention head %d", it, h);
  }
  /* GEMV */
  const int d_in = 1 + rnd(300), d_out = 1 + rnd(300), rows = 1 + rnd(4);
  float* x = xmalloc(sizeof(float) * (size_t)rows * d_in);
  uint16_t* W = xmalloc(2u * (size_t)d_in * d_out);
  float* y = xmalloc(sizeof(float) * (size_t)rows * d_out);
  for (size_t i = 0; i < (size_t)rows * d_in; i++) x[i] = frnd();
  for (size_t i = 0; i < (size_t)d_in * d_out; i++) W[i] = oracle_f32_to_f16(frnd());
  oracle_matvec(x, W, y, d_in, d_out, rows, 0);
  for (int m = 0; m < rows; m++)
    for (int c = 0; c < d_out; c++) {
      double s = 0, a = 0;
      for (int r = 0; r < d_in; r++) {
        const double t = (double)x[(size_t)m * d_in + r] *
                         (double)oracle_f16_to_f32(W[(size_t)r * d_out + c]);
        s += t;
        a += fabs(t);
      }
      CHECK(fabs((double)y[(size_t)m * d_out + c] - s) <= 1e-6 * a + 1e-30,
            "case %d: matvec (%d, %d)", it, m, c);
    }
  free(x);
  free(W);
  free(y);
  free(q);
  free(out);
  free(ref);
  free(kg);
  free(vg);
  free(k);
  free(v);
  free(perm);
  free(pool);
}

int main(int argc, char** argv) {
  const int cases = argc > 1 ? atoi(argv[1]) : 300;
  if (argc > 2) g_state ^= (uint64_t)atoll(argv[2]);
  check_f16();
  for (int i = 0; i < cases; i++) check_case(i);
  if (g_fail) {
    fprintf(stderr, "%d failures\n", g_fail);
    return 1;
  }
  printf("oracle check: %d cases, all checks passed\n", cases);
  return 0;
}
