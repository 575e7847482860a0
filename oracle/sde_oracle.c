/*
 * sde_oracle.c — CPU restatement of the reference's paged-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or the timed CPU baseline).  The product path never calls it.
 *
 * Each function cites the reference file:line it restates
 * (arkhamHack/speculative_decode_engine, cuda/...).  The reference itself
 * is CUDA C++ (nvcc, cuda_fp16.h, cooperative groups, cuBLAS) and cannot be
 * compiled in this image, so there is no oracle/_ref build.
 *
 * Pinning (tests/test_oracle.py): fp16 conversion against numpy's IEEE
 * float16 cast; append/gather against a numpy byte model and permutation /
 * contiguous-layout invariants; the tiled attention against an independent
 * fp64 brute force, torch's scaled_dot_product_attention, and closed-form
 * special cases (L=1, uniform logits, one-hot logits, total_len=0).
 */
#include <float.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- fp16 <-> fp32 (IEEE 754 binary16), written from the format spec ---- */

/* fp32 -> fp16 bits, round to nearest, ties to even (what __float2half does,
 * kv_cache.cu:89-90).  NaN keeps its sign and becomes a quiet NaN. */
uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) { /* inf or nan */
    if (man == 0) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | (man >> 13));
  }
  int e = (int)exp - 127 + 15; /* rebias */
  if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
  if (e <= 0) {
    /* subnormal (or zero) in fp16: value = man_full * 2^(exp-150);
     * fp16 subnormal unit is 2^-24, so shift = 126 - exp. */
    if (e < -10) return (uint16_t)sign; /* below half the smallest subnormal */
    uint32_t full = man | 0x800000u;
    int shift = 14 - e; /* = 126 - exp, in [14, 24] */
    uint32_t q = full >> shift;
    uint32_t rem = full & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q); /* q may carry into the normal range */
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* may carry to inf */
  return (uint16_t)(sign | q);
}

/* fp16 bits -> fp32, exact (what __half2float does, kv_cache.cu:110-111). */
float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t man = (uint32_t)h & 0x3ffu;
  uint32_t x;
  if (exp == 0) {
    if (man == 0) {
      x = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do { man <<= 1; e++; } while (!(man & 0x400u));
      man &= 0x3ffu;
      x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    x = sign | 0x7f800000u | (man << 13);
  } else {
    x = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

void oracle_f32_to_f16_array(const float* src, uint16_t* dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = oracle_f32_to_f16(src[i]);
}

void oracle_f16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = oracle_f16_to_f32(src[i]);
}

/* ---- paged layout (kv_cache.h:5-18, kv_cache.cu:58-68) ------------------ */

/* Element offset of K[pos] (is_v = 0) or V[pos] (is_v = 1) in the pool:
 * block_ptr = pool + phys * 2*BS*kv_dim (size_t, kv_cache.cu:58-62);
 * K row at slot*kv_dim, V row at BS*kv_dim + slot*kv_dim (kv_cache.cu:83-85). */
static size_t row_offset(const int32_t* table, int kv_dim, int bs, int pos,
                         int is_v) {
  int lb = pos / bs;
  int slot = pos % bs;
  size_t phys = (size_t)table[lb];
  return phys * 2u * (size_t)bs * (size_t)kv_dim +
         (size_t)(is_v ? bs : 0) * (size_t)kv_dim + (size_t)slot * (size_t)kv_dim;
}

/* cublas_kv_append_kernel (kernels.cu:826-844) == kv_cache_append repeated
 * (kv_cache.cu:70-93): token m goes to pos_base+m; fp32 -> fp16 RNE. */
void oracle_kv_append(uint16_t* pool, const int32_t* table, int kv_dim, int bs,
                      const float* k, const float* v, int pos_base, int n) {
  for (int m = 0; m < n; m++) {
    int pos = pos_base + m;
    uint16_t* kd = pool + row_offset(table, kv_dim, bs, pos, 0);
    uint16_t* vd = pool + row_offset(table, kv_dim, bs, pos, 1);
    for (int i = 0; i < kv_dim; i++) {
      kd[i] = oracle_f32_to_f16(k[(size_t)m * kv_dim + i]);
      vd[i] = oracle_f32_to_f16(v[(size_t)m * kv_dim + i]);
    }
  }
}

/* Raw fp16 rows written without conversion (the prefill helper). */
void oracle_kv_write_fp16(uint16_t* pool, const int32_t* table, int kv_dim,
                          int bs, const uint16_t* k, const uint16_t* v,
                          int pos_base, int n) {
  for (int m = 0; m < n; m++) {
    int pos = pos_base + m;
    memcpy(pool + row_offset(table, kv_dim, bs, pos, 0), k + (size_t)m * kv_dim,
           (size_t)kv_dim * 2u);
    memcpy(pool + row_offset(table, kv_dim, bs, pos, 1), v + (size_t)m * kv_dim,
           (size_t)kv_dim * 2u);
  }
}

/* kv_cache_read (kv_cache.cu:95-114) for positions pos..pos+n-1. */
void oracle_kv_gather(const uint16_t* pool, const int32_t* table, int kv_dim,
                      int bs, int pos, int n, float* k, float* v) {
  for (int m = 0; m < n; m++) {
    const uint16_t* ks = pool + row_offset(table, kv_dim, bs, pos + m, 0);
    const uint16_t* vs = pool + row_offset(table, kv_dim, bs, pos + m, 1);
    for (int i = 0; i < kv_dim; i++) {
      k[(size_t)m * kv_dim + i] = oracle_f16_to_f32(ks[i]);
      v[(size_t)m * kv_dim + i] = oracle_f16_to_f32(vs[i]);
    }
  }
}

/* ---- attention ----------------------------------------------------------- */

/* Literal restatement of device_flash_attention_gqa for ONE query head
 * (attention.h:21-127 with the head loop of :35 hoisted to the caller):
 * tiles of bs positions; logits = (q . K[p]) * dph^-1/2 (:49-66); tile max,
 * alpha = expf(m_prev - m_new) except on the first tile (:70-87); rescale
 * the accumulator (:91-94); add sum_p expf(logit_p - m_new) V[p] (:98-115);
 * finally multiply by 1/l when l > 1e-20 and finite, else 0 (:120-126).
 * fp32 arithmetic with libm expf (the reference uses fast-math expf). */
static void tiled_one_head(const float* q, float* out, const uint16_t* pool,
                           const int32_t* table, int kv_dim, int bs, int dph,
                           int kv_off, int total_len) {
  const float scale = 1.0f / sqrtf((float)dph);
  const int n_logical = (total_len + bs - 1) / bs;
  float logits[1024];
  float s_m = -FLT_MAX, s_l = 0.f;
  for (int e = 0; e < dph; e++) out[e] = 0.f;
  for (int lb = 0; lb < n_logical; lb++) {
    const int p0 = lb * bs;
    for (int sl = 0; sl < bs; sl++) {
      int p = p0 + sl;
      float logit = -FLT_MAX;
      if (p < total_len) {
        const uint16_t* ks = pool + row_offset(table, kv_dim, bs, p, 0) + kv_off;
        float dot = 0.f;
        for (int e = 0; e < dph; e++) dot += q[e] * oracle_f16_to_f32(ks[e]);
        logit = dot * scale;
      }
      logits[sl] = logit;
    }
    float m_tile = -FLT_MAX;
    for (int sl = 0; sl < bs; sl++)
      if (p0 + sl < total_len) m_tile = fmaxf(m_tile, logits[sl]);
    float m_prev = s_m;
    float m_new = fmaxf(m_prev, m_tile);
    float alpha = (lb > 0) ? expf(m_prev - m_new) : 1.f;
    float l_tile = 0.f;
    for (int sl = 0; sl < bs; sl++) {
      if (p0 + sl >= total_len) continue;
      l_tile += expf(logits[sl] - m_new);
    }
    s_m = m_new;
    s_l = alpha * s_l + l_tile;
    for (int e = 0; e < dph; e++) out[e] *= alpha;
    for (int e = 0; e < dph; e++) {
      float acc = 0.f;
      for (int sl = 0; sl < bs; sl++) {
        int p = p0 + sl;
        if (p >= total_len) continue;
        float w = expf(logits[sl] - m_new);
        const uint16_t* vs = pool + row_offset(table, kv_dim, bs, p, 1) + kv_off;
        acc += w * oracle_f16_to_f32(vs[e]);
      }
      out[e] += acc;
    }
  }
  float inv = (s_l > 1e-20f && isfinite(s_l)) ? (1.f / s_l) : 0.f;
  for (int e = 0; e < dph; e++) out[e] *= inv;
}

/* Textbook softmax(q K^T dph^-1/2) V in fp64 over the gathered keys
 * (no tiling, no online rescaling): an independent formulation. */
static void f64_one_head(const float* q, double* out, const uint16_t* pool,
                         const int32_t* table, int kv_dim, int bs, int dph,
                         int kv_off, int total_len) {
  const double scale = 1.0 / sqrt((double)dph);
  double mx = -INFINITY;
  for (int e = 0; e < dph; e++) out[e] = 0.0;
  if (total_len <= 0) return;
  /* two passes: max, then weights (keeps memory O(dph)) */
  for (int p = 0; p < total_len; p++) {
    const uint16_t* ks = pool + row_offset(table, kv_dim, bs, p, 0) + kv_off;
    double dot = 0.0;
    for (int e = 0; e < dph; e++) dot += (double)q[e] * oracle_f16_to_f32(ks[e]);
    dot *= scale;
    if (dot > mx) mx = dot;
  }
  double den = 0.0;
  for (int p = 0; p < total_len; p++) {
    const uint16_t* ks = pool + row_offset(table, kv_dim, bs, p, 0) + kv_off;
    const uint16_t* vs = pool + row_offset(table, kv_dim, bs, p, 1) + kv_off;
    double dot = 0.0;
    for (int e = 0; e < dph; e++) dot += (double)q[e] * oracle_f16_to_f32(ks[e]);
    double w = exp(dot * scale - mx);
    den += w;
    for (int e = 0; e < dph; e++) out[e] += w * oracle_f16_to_f32(vs[e]);
  }
  for (int e = 0; e < dph; e++) out[e] /= den;
}

/* device_flash_attention_gqa over all heads for one query with an explicit
 * total_len (attention.h:21-37): head h reads KV head h*nkv/nh. */
void oracle_attention_tiled(const float* q_all, float* out, const uint16_t* pool,
                            const int32_t* table, int kv_dim, int bs, int nh,
                            int nkv, int dph, int total_len) {
  for (int h = 0; h < nh; h++) {
    int kv_head = h * nkv / nh;
    tiled_one_head(q_all + (size_t)h * dph, out + (size_t)h * dph, pool, table,
                   kv_dim, bs, dph, kv_head * dph, total_len);
  }
}

void oracle_attention_f64(const float* q_all, double* out, const uint16_t* pool,
                          const int32_t* table, int kv_dim, int bs, int nh,
                          int nkv, int dph, int total_len) {
  for (int h = 0; h < nh; h++) {
    int kv_head = h * nkv / nh;
    f64_one_head(q_all + (size_t)h * dph, out + (size_t)h * dph, pool, table,
                 kv_dim, bs, dph, kv_head * dph, total_len);
  }
}

/* cublas_attention_kernel (kernels.cu:904-940): query m of a window of M
 * sees total_len = pos_base + m + 1 keys (kernels.cu:915).  q/out are
 * [M][nh*dph].  mode 0: tiled fp32 restatement (out fp32); mode 1: fp64
 * brute force (out_f64).  The (m, h) pairs are independent and run on up to
 * n_threads OpenMP threads (1 = serial).  Returns the thread count used. */
int oracle_paged_attention(const float* q, float* out, double* out_f64,
                           const uint16_t* pool, const int32_t* table,
                           int kv_dim, int bs, int nh, int nkv, int dph,
                           int pos_base, int M, int mode, int n_threads) {
  int used = 1;
  const int pairs = M * nh;
#ifdef _OPENMP
  if (n_threads < 1) n_threads = 1;
  used = n_threads;
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads)
#endif
  for (int i = 0; i < pairs; i++) {
    int m = i / nh, h = i % nh;
    int kv_head = h * nkv / nh;
    int total_len = pos_base + m + 1;
    size_t off = (size_t)m * nh * dph + (size_t)h * dph;
    if (mode == 0)
      tiled_one_head(q + off, out + off, pool, table, kv_dim, bs, dph,
                     kv_head * dph, total_len);
    else
      f64_one_head(q + off, out_f64 + off, pool, table, kv_dim, bs, dph,
                   kv_head * dph, total_len);
  }
  return used;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* device_matvec_partial_accum / device_matvec_partial (utils.h:417-452),
 * literally: for each output column c (one thread per column in the
 * reference), acc = sum over r = 0..d_in-1 of x[r] * float(W[r*d_out + c])
 * in row order, fp32, multiply-add fused (nvcc contracts `acc += a*b`), then
 * out[c] = acc or out[c] += acc.  For n_rows rows of x (device_matvec_batched,
 * utils.h:248-267, is the same per row).  Columns are independent, so the
 * OpenMP split over columns keeps the reference's per-column order. */
void oracle_matvec(const float* x, const uint16_t* W, float* out, int d_in, int d_out,
                   int n_rows, int accumulate) {
  for (int m = 0; m < n_rows; m++) {
    const float* xm = x + (size_t)m * d_in;
    float* om = out + (size_t)m * d_out;
#pragma omp parallel for schedule(static)
    for (int c = 0; c < d_out; c++) {
      float acc = 0.f;
      for (int r = 0; r < d_in; r++)
        acc = fmaf(xm[r], oracle_f16_to_f32(W[(size_t)r * d_out + c]), acc);
      om[c] = accumulate ? om[c] + acc : acc;
    }
  }
}
