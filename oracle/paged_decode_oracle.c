/*
 * paged_decode_oracle.c -- C restatement of paged decode attention.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (checker at sizes numpy is too
 * slow for), __graft_entry__.smoke() and bench.py's cpu_baseline leg (the
 * timed CPU baseline). Never part of the product path.
 *
 * Restates paged_attention_batch_online_v1
 * (minivllm/paged_attention_batch.py:121-278) one (b, h) pair at a time:
 * for each logical block j < ceil(ctx/S) of table row b, with n valid slots,
 *   s_t   = scale * q . K[t]                  t < n
 *   m'    = max(m, max_t s_t)
 *   alpha = exp(m - m'),  p_t = exp(s_t - m')
 *   l'    = alpha * l + sum_t p_t
 *   O'    = (alpha * l * O + sum_t p_t V[t]) / l'
 * Slots past the context are never read. A table entry outside [0, N) inside
 * the context is skipped (the HIP kernel's bounds rule; the reference asserts
 * it never happens). ctx == 0 gives O = 0.
 *
 * Layouts: q [B, H, D] and pool [L, N, S, H, D], contiguous; dtype 0 = f32,
 * 1 = bfloat16 bit patterns. Arithmetic in double (acc_double = 1, the
 * checker) or float (acc_double = 0, the fp32 recurrence of the reference).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

static inline float load_elem(const void* base, int dtype, int64_t i) {
  return dtype == 1 ? bf16_to_f32(((const uint16_t*)base)[i]) : ((const float*)base)[i];
}

#define DEFINE_PAIR(NAME, ACC)                                                              \
  static void NAME(const void* q, const void* kp, const void* vp, int dtype,              \
                   const int64_t* tables, int64_t ctx, int64_t b, int64_t h, int64_t H,   \
                   int64_t D, int64_t S, int64_t N, int64_t M, int64_t layer_off,         \
                   double scale, float* out_row) {                                        \
    ACC qv[1024], O[1024], s[1024], p[1024];                                               \
    for (int64_t d = 0; d < D; ++d) {                                                       \
      qv[d] = (ACC)load_elem(q, dtype, (b * H + h) * D + d);                               \
      O[d] = 0;                                                                             \
    }                                                                                       \
    ACC m = -INFINITY, l = 0;                                                               \
    const int64_t nblk = (ctx + S - 1) / S;                                                 \
    for (int64_t j = 0; j < nblk && j < M; ++j) {                                           \
      const int64_t phys = tables[b * M + j];                                               \
      if (phys < 0 || phys >= N) continue;                                                  \
      const int64_t n = ctx - j * S < S ? ctx - j * S : S;                                  \
      ACC bmax = -INFINITY;                                                                 \
      for (int64_t t = 0; t < n; ++t) {                                                     \
        const int64_t row = layer_off + ((phys * S + t) * H + h) * D;                       \
        ACC acc = 0;                                                                        \
        for (int64_t d = 0; d < D; ++d) acc += qv[d] * (ACC)load_elem(kp, dtype, row + d);  \
        s[t] = acc * (ACC)scale;                                                            \
        if (s[t] > bmax) bmax = s[t];                                                       \
      }                                                                                     \
      const ACC mn = m > bmax ? m : bmax;                                                   \
      const ACC alpha = (m == -INFINITY) ? (ACC)0 : (ACC)exp((double)(m - mn));             \
      ACC psum = 0;                                                                         \
      for (int64_t t = 0; t < n; ++t) {                                                     \
        p[t] = (ACC)exp((double)(s[t] - mn));                                               \
        psum += p[t];                                                                       \
      }                                                                                     \
      const ACC ln = alpha * l + psum;                                                      \
      for (int64_t d = 0; d < D; ++d) {                                                     \
        ACC pv = 0;                                                                         \
        for (int64_t t = 0; t < n; ++t)                                                     \
          pv += p[t] * (ACC)load_elem(vp, dtype, layer_off + ((phys * S + t) * H + h) * D + d); \
        O[d] = (alpha * l * O[d] + pv) / ln;                                                \
      }                                                                                     \
      m = mn;                                                                               \
      l = ln;                                                                               \
    }                                                                                       \
    for (int64_t d = 0; d < D; ++d) out_row[d] = (float)O[d];                               \
  }

DEFINE_PAIR(pair_f64, double)
DEFINE_PAIR(pair_f32, float)

/* Returns 0, or -1 on an argument it cannot handle (D > 1024, S > 1024). */
int oracle_paged_decode(const void* q, const void* k_pool, const void* v_pool, int dtype,
                        const int64_t* block_tables, const int64_t* context_lens, int64_t B,
                        int64_t H, int64_t D, int64_t S, int64_t N, int64_t M, int64_t L,
                        int64_t layer, double scale, int acc_double, float* out, int nthreads) {
  if (D > 1024 || S > 1024 || layer < 0 || layer >= L || (dtype != 0 && dtype != 1)) return -1;
  const int64_t layer_off = layer * N * S * H * D;
  const int64_t pairs = B * H;
  if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (int64_t i = 0; i < pairs; ++i) {
    const int64_t b = i / H, h = i % H;
    int64_t ctx = context_lens[b];
    if (ctx < 0) ctx = 0;
    if (ctx > M * S) ctx = M * S;
    float* row = out + i * D;
    if (acc_double)
      pair_f64(q, k_pool, v_pool, dtype, block_tables, ctx, b, h, H, D, S, N, M, layer_off, scale, row);
    else
      pair_f32(q, k_pool, v_pool, dtype, block_tables, ctx, b, h, H, D, S, N, M, layer_off, scale, row);
  }
  return 0;
}
